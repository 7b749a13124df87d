// The checks of the reference's tests/test_cuda_quant_kernel_parity.cpp, run
// through the HIP backend's reference interface (hip_backend.h): for Q4_K,
// Q5_0 and Q8_0, the crafted blocks of test_cuda_quant_kernel_parity.cpp:26-67
// (one element -1 per block, every row the same block) times a ones vector,
// within its bar (max abs difference 1e-3), for
//   - hip_backend_matmul (B quantized along its rows) against cpu_matmul, and
//   - hip_backend_matmul_rhs_transposed (the decode GEMV) against the
//     reference dispatcher backend_matmul_rhs_transposed on its CPU path;
// then the same two products on seeded random blocks at a decode shape
// (K = 4096), within the GEMV tolerance |err| <= 1e-3 |ref| + 1e-4 max |ref|.
// The expected side is the reference's CPU code (oracle/_ref/libmxref.so).
#include <cmath>
#include <cstdint>
#include <cstring>
#include <iostream>
#include <random>
#include <string>
#include <vector>

#include "backend/backend_runtime.h"
#include "backend/cpu/cpu_backend.h"
#include "hip_backend.h"
#include "tensor/tensor.h"

namespace {

struct Format {
    DataType type;
    const char* name;
    size_t elems, bytes;
};

const Format kFormats[] = {
    {DataType::Q4_K, "Q4_K", TENSOR_Q4_K_QK_K, TENSOR_Q4_K_BLOCK_SIZE},
    {DataType::Q5_0, "Q5_0", TENSOR_Q5_0_QK, TENSOR_Q5_0_BLOCK_SIZE},
    {DataType::Q8_0, "Q8_0", TENSOR_Q8_0_QK, TENSOR_Q8_0_BLOCK_SIZE},
};

Tensor* make_quant(const Format& f, size_t rows, size_t cols, const std::vector<uint8_t>& packed) {
    switch (f.type) {
    case DataType::Q4_K: return tensor_create_q4_k_from_bytes(rows, cols, packed.data(), packed.size());
    case DataType::Q5_0: return tensor_create_q5_0_from_bytes(rows, cols, packed.data(), packed.size());
    default: return tensor_create_q8_0_from_bytes(rows, cols, packed.data(), packed.size());
    }
}

// the reference test's blocks: scale(s) 1.0 and one element decoding to -1
std::vector<uint8_t> crafted_block(const Format& f) {
    std::vector<uint8_t> b(f.bytes, 0);
    const uint16_t one = 0x3c00;
    std::memcpy(b.data(), &one, 2);
    if (f.type == DataType::Q4_K) {
        std::memcpy(b.data() + 2, &one, 2);
        b[4 + 4] = 0x40;
        b[4 + 8] = 0x10;
        b[16 + 64] = 0x01;
    } else if (f.type == DataType::Q5_0) {
        b[2 + 4] = 0x0f;  // element 0: 15 - 16
    } else {
        b[2] = 0xff;  // element 0: int8 -1
    }
    return b;
}

// finite binary16 of magnitude 2^-10 .. 2^-6 and random mantissa
uint16_t small_half(std::mt19937& g) { return (uint16_t)(((5 + g() % 5) << 10) | (g() % 1024)); }

std::vector<uint8_t> random_blocks(const Format& f, size_t nblocks, std::mt19937& g) {
    std::vector<uint8_t> p(nblocks * f.bytes);
    for (auto& v : p) v = (uint8_t)g();
    for (size_t i = 0; i < nblocks; ++i) {
        uint8_t* b = p.data() + i * f.bytes;
        const uint16_t d = small_half(g), m = small_half(g);
        std::memcpy(b, &d, 2);
        if (f.type == DataType::Q4_K) std::memcpy(b + 2, &m, 2);
    }
    return p;
}

double max_abs(const float* a, const float* b, size_t n) {
    double m = 0.0;
    for (size_t i = 0; i < n; ++i) m = std::fmax(m, std::fabs((double)a[i] - (double)b[i]));
    return m;
}

// |got - want| <= rtol |want| + floor * max |want|, elementwise
bool within(const float* got, const float* want, size_t n, double rtol, double floor) {
    double scale = 0.0;
    for (size_t i = 0; i < n; ++i) scale = std::fmax(scale, std::fabs((double)want[i]));
    for (size_t i = 0; i < n; ++i) {
        const double d = std::fabs((double)got[i] - (double)want[i]);
        if (d > rtol * std::fabs((double)want[i]) + floor * scale) {
            std::cerr << "    [" << i << "] got " << got[i] << ", want " << want[i] << "\n";
            return false;
        }
    }
    return true;
}

// K x N with identical crafted rows, ones vector: the reference test's case
bool crafted_case(const Format& f) {
    const size_t K = f.elems, N = f.elems;
    const std::vector<uint8_t> blk = crafted_block(f);
    std::vector<uint8_t> packed;
    for (size_t r = 0; r < K; ++r) packed.insert(packed.end(), blk.begin(), blk.end());
    Tensor* A = tensor_create_f32(1, K);
    Tensor* Bq = make_quant(f, K, N, packed);
    Tensor* C_cpu = tensor_create_f32(1, N);
    Tensor* C_hip = tensor_create_f32(1, N);
    if (!A || !Bq || !C_cpu || !C_hip) return false;
    for (size_t i = 0; i < K; ++i) static_cast<float*>(A->data)[i] = 1.0f;

    bool ok = true;
    // A . B (B along its rows)
    if (!cpu_matmul(A, Bq, C_cpu) || !hip_backend_matmul(A, Bq, C_hip)) {
        std::cout << "  x matmul failed: " << hip_backend_last_error_msg() << "\n";
        ok = false;
    } else {
        const double d = max_abs(static_cast<float*>(C_hip->data), static_cast<float*>(C_cpu->data), N);
        std::cout << "  " << f.name << " matmul          max abs diff " << d << "\n";
        ok = d <= 1e-3;
    }
    // A . B^T (B's rows are the weight rows)
    if (!backend_matmul_rhs_transposed(A, Bq, C_cpu) || !hip_backend_matmul_rhs_transposed(A, Bq, C_hip)) {
        std::cout << "  x matmul_rhs_transposed failed: " << hip_backend_last_error_msg() << "\n";
        ok = false;
    } else {
        const double d = max_abs(static_cast<float*>(C_hip->data), static_cast<float*>(C_cpu->data), N);
        std::cout << "  " << f.name << " rhs_transposed  max abs diff " << d << "\n";
        ok = ok && d <= 1e-3;
    }
    tensor_free(A);
    tensor_free(Bq);
    tensor_free(C_cpu);
    tensor_free(C_hip);
    return ok;
}

// seeded random blocks at a decode shape: rhs_transposed with K = 4096 and
// 96 weight rows; matmul with 64 rows of 512 columns
bool random_case(const Format& f, uint32_t seed) {
    std::mt19937 g(seed);
    bool ok = true;
    {
        const size_t K = 4096, N = 96;
        const std::vector<uint8_t> packed = random_blocks(f, N * (K / f.elems), g);
        Tensor* A = tensor_create_f32(1, K);
        Tensor* Bq = make_quant(f, N, K, packed);
        Tensor* C_cpu = tensor_create_f32(1, N);
        Tensor* C_hip = tensor_create_f32(1, N);
        if (!A || !Bq || !C_cpu || !C_hip) return false;
        std::normal_distribution<float> nd(0.f, 1.f);
        for (size_t i = 0; i < K; ++i) static_cast<float*>(A->data)[i] = nd(g);
        ok = backend_matmul_rhs_transposed(A, Bq, C_cpu) && hip_backend_matmul_rhs_transposed(A, Bq, C_hip) &&
             within(static_cast<float*>(C_hip->data), static_cast<float*>(C_cpu->data), N, 1e-3, 1e-4);
        std::cout << "  " << (ok ? "✓ " : "✗ ") << f.name << " random rhs_transposed 96 x 4096\n";
        tensor_free(A);
        tensor_free(Bq);
        tensor_free(C_cpu);
        tensor_free(C_hip);
    }
    {
        const size_t K = 64, N = 512;
        const std::vector<uint8_t> packed = random_blocks(f, K * (N / f.elems), g);
        Tensor* A = tensor_create_f32(1, K);
        Tensor* Bq = make_quant(f, K, N, packed);
        Tensor* C_cpu = tensor_create_f32(1, N);
        Tensor* C_hip = tensor_create_f32(1, N);
        if (!A || !Bq || !C_cpu || !C_hip) return false;
        std::normal_distribution<float> nd(0.f, 1.f);
        for (size_t i = 0; i < K; ++i) static_cast<float*>(A->data)[i] = nd(g);
        const bool mm = cpu_matmul(A, Bq, C_cpu) && hip_backend_matmul(A, Bq, C_hip) &&
                        within(static_cast<float*>(C_hip->data), static_cast<float*>(C_cpu->data), N, 1e-4, 1e-5);
        std::cout << "  " << (mm ? "✓ " : "✗ ") << f.name << " random matmul 64 x 512\n";
        ok = ok && mm;
        tensor_free(A);
        tensor_free(Bq);
        tensor_free(C_cpu);
        tensor_free(C_hip);
    }
    return ok;
}

}  // namespace

int main(int argc, char** argv) {
    const bool require = argc > 1 && std::string(argv[1]) == "--require-device";
    std::cout << "[TEST] HIP quant kernel parity (reference interface)" << std::endl;
    if (!hip_backend_is_available()) {
        std::cout << "HIP not available (" << hip_backend_last_error_msg() << "); skipping test" << std::endl;
        return require ? 7 : 0;
    }
    bool all_ok = true;
    uint32_t seed = 0x5eed0100u;
    for (const Format& f : kFormats) {
        std::cout << "\n[TEST] Format: " << f.name << std::endl;
        all_ok = crafted_case(f) && all_ok;
        all_ok = random_case(f, seed++) && all_ok;
    }
    hip_backend_release_resources();
    return all_ok ? 0 : 6;
}
