// The four vector operations of the reference's backend interface
// (cuda_backend.h:26-29) through hip_backend.h, against the reference's own
// CPU versions (cpu_backend.cpp:325-393, in oracle/_ref/libmxref.so) on
// seeded data, with the allclose bar of the reference's matmul test
// (rtol 1e-3, atol 1e-4).  Shapes follow the attention call sites
// (transformer.cpp:575, :583, :617): head_dim 128 rows of a KV cache with a
// row stride wider than K, a ring that wraps, and the V-weighted column sum.
// Empty inputs return false, as the CPU versions do.
#include <cmath>
#include <cstdint>
#include <iostream>
#include <random>
#include <string>
#include <vector>

#include "backend/cpu/cpu_backend.h"
#include "hip_backend.h"

namespace {

bool allclose(const std::vector<float>& got, const std::vector<float>& want, const char* what) {
    for (size_t i = 0; i < want.size(); ++i) {
        const float d = std::fabs(got[i] - want[i]);
        if (d > 1e-4f && d > 1e-3f * std::fabs(want[i])) {
            std::cout << "  ✗ " << what << ": [" << i << "] got " << got[i] << ", want " << want[i] << std::endl;
            return false;
        }
    }
    std::cout << "  ✓ " << what << std::endl;
    return true;
}

std::vector<float> randn(size_t n, std::mt19937& g) {
    std::normal_distribution<float> nd(0.f, 1.f);
    std::vector<float> v(n);
    for (auto& x : v) x = nd(g);
    return v;
}

}  // namespace

int main(int argc, char** argv) {
    const bool require = argc > 1 && std::string(argv[1]) == "--require-device";
    std::cout << "[TEST] HIP vector ops (reference interface)" << std::endl;
    if (!hip_backend_is_available()) {
        std::cout << "HIP not available (" << hip_backend_last_error_msg() << "); skipping test" << std::endl;
        return require ? 7 : 0;
    }
    std::mt19937 g(0x5eed0200u);
    bool ok = true;
    const size_t K = 128, stride = 1024 + 8;  // one kv head's dims inside wider cache rows

    {   // dot of q with 600 cached rows
        const size_t n = 600;
        const std::vector<float> q = randn(K, g), rows = randn((n - 1) * stride + K, g);
        std::vector<float> want(n), got(n, NAN);
        ok = cpu_vec_dot_rows(q.data(), rows.data(), want.data(), K, n, stride) &&
             hip_backend_vec_dot_rows(q.data(), rows.data(), got.data(), K, n, stride) &&
             allclose(got, want, "vec_dot_rows 600 x 128, stride 1032") && ok;
    }
    {   // ring of 512 slots, 500 live rows starting at slot 300 (wraps)
        const size_t seq_max = 512, len = 500, head = 300;
        const std::vector<float> q = randn(K, g), ring = randn((seq_max - 1) * stride + K, g);
        std::vector<float> want(len), got(len, NAN);
        ok = cpu_vec_dot_rows_ring(q.data(), ring.data(), head, seq_max, len, K, stride, want.data()) &&
             hip_backend_vec_dot_rows_ring(q.data(), ring.data(), head, seq_max, len, K, stride, got.data()) &&
             allclose(got, want, "vec_dot_rows_ring head 300, 500 of 512") && ok;
    }
    {   // softmax weights times 600 value rows
        const size_t n = 600;
        const std::vector<float> p = randn(n, g), rows = randn((n - 1) * stride + K, g);
        std::vector<float> want(K), got(K, NAN);
        ok = cpu_vec_mul_rows_cols(p.data(), rows.data(), want.data(), n, K, stride) &&
             hip_backend_vec_mul_rows_cols(p.data(), rows.data(), got.data(), n, K, stride) &&
             allclose(got, want, "vec_mul_rows_cols 600 x 128, stride 1032") && ok;
    }
    {   // x^T W with W 1024 x 3000 inside rows of 3072
        const size_t k = 1024, n = 3000, st = 3072;
        const std::vector<float> x = randn(k, g), w = randn((k - 1) * st + n, g);
        std::vector<float> want(n), got(n, NAN);
        ok = cpu_matvec_strided(x.data(), w.data(), want.data(), k, n, st) &&
             hip_backend_matvec_strided(x.data(), w.data(), got.data(), k, n, st) &&
             allclose(got, want, "matvec_strided 1024 x 3000, stride 3072") && ok;
    }
    {   // empty inputs: false on both sides
        std::vector<float> v(4, 1.f), o(4);
        const bool rejected = !hip_backend_vec_dot_rows(v.data(), v.data(), o.data(), 0, 1, 4) &&
                              !hip_backend_vec_dot_rows_ring(v.data(), v.data(), 0, 1, 0, 4, 4, o.data()) &&
                              !hip_backend_vec_mul_rows_cols(v.data(), v.data(), o.data(), 0, 4, 4) &&
                              !cpu_vec_dot_rows(v.data(), v.data(), o.data(), 0, 1, 4);
        std::cout << (rejected ? "  ✓ empty inputs rejected" : "  ✗ an empty input was accepted") << std::endl;
        ok = rejected && ok;
    }
    hip_backend_release_resources();
    std::cout << "Test finished" << std::endl;
    return ok ? 0 : 1;
}
