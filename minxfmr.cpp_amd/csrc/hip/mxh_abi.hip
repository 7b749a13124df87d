// mxh_abi.hip — the extern "C" surface declared in include/minxfmr_hip.h.
//
// Holds the per-process device context (device, stream, timing events, the
// weight cache of the per-op interface) and validates every request on the
// host before any kernel sees it: a launch that reaches the device has shapes
// the kernel's indexing assumes.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <utility>

#include "mxh_internal.h"

namespace mxh {
namespace {

struct Context {
    bool ready = false;
    int device = -1;
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    // per-op interface: weights cached by (host pointer, bytes)
    std::map<std::pair<const void*, size_t>, void*> weights;
    // grow-only staging buffers for host-pointer ops
    void* stage[4] = {nullptr, nullptr, nullptr, nullptr};
    size_t stage_bytes[4] = {0, 0, 0, 0};
};

Context g_ctx;
thread_local std::string g_err;

// Device scratch of mxh_gemm_q_f16_noalloc: the staged activations (fp16 hi
// and lo of a 2^e, the split sub-block sums, 2^-e per row).  Each GPU holds
// its own copy from module load until the process ends; in host code the
// array's name is only a stand-in, so kernels get the device address that
// hipGetSymbolAddress returned for the current device (g_scratch_ptr).
constexpr size_t kNoallocScratchBytes = 12u << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) uint8_t scratch[kNoallocScratchBytes];
void* g_scratch_ptr[kMaxDevices] = {};

// staging bytes of an m x k activation block in the layout of f16_rows_layout
size_t f16_rows_bytes(size_t m, size_t k) { return 4 * m * k + 4 * (m * k / 32) + 4 * m; }

struct F16Rows {
    uint16_t *a_hi, *a_lo, *s_hi, *s_lo;
    float* rscale;
};
F16Rows f16_rows_layout(void* buf, size_t m, size_t k) {
    const size_t mk = m * k, nsb = mk / 32;
    F16Rows r;
    r.a_hi = static_cast<uint16_t*>(buf);
    r.a_lo = r.a_hi + mk;
    r.s_hi = r.a_lo + mk;
    r.s_lo = r.s_hi + nsb;
    r.rscale = reinterpret_cast<float*>(r.s_lo + nsb);
    return r;
}

int ensure_ready() {
    if (g_ctx.ready) return MXH_OK;
    return mxh_init(0);
}

// validation and the two launches of mxh_gemm_q_f16 over staging at `buf`
int gemm_q_f16_body(const char* who, int type, const float* a, int64_t m, const void* w, int64_t n, int64_t k,
                    float* out, int form, void* buf) {
    const F16Rows r = f16_rows_layout(buf, (size_t)m, (size_t)k);
    if (int rc = rows_to_f16_launch(a, (int)k, nullptr, 0.f, (int)k, r.a_hi, r.a_lo, (int)k, r.s_hi, r.s_lo,
                                    (int)k / 32, r.rscale, (int)m, g_ctx.stream))
        return set_error(rc, "%s: conversion launch", who);
    if (int rc = gemm_q_f16_run(type, r.a_hi, r.a_lo, (int)k, r.s_hi, r.s_lo, (int)k / 32, r.rscale, w, out, (int)n,
                                nullptr, (int)m, (int)n, (int)k, form, nullptr, 0, g_ctx.stream))
        return set_error(rc, "%s: launch", who);
    return check_hip(hipGetLastError(), who);
}

int gemm_q_f16_check(const char* who, int type, const float* a, int64_t m, const void* w, int64_t n, int64_t k,
                     float* out) {
    if (!a || !w || !out) return set_error(MXH_ERR_ARG, "%s: null pointer", who);
    if (m <= 0 || n <= 0 || k <= 0 || m > INT32_MAX || n > INT32_MAX || k > INT32_MAX ||
        !gemm_q_f16_supported(type, (int)k))
        return set_error(MXH_ERR_ARG, "%s: bad shape %lldx%lldx%lld for type %d", who, (long long)m, (long long)n,
                         (long long)k, type);
    if (((uintptr_t)w & 15) || ((uintptr_t)a & 15))
        return set_error(MXH_ERR_ARG, "%s: a and w must be 16-byte aligned", who);
    return MXH_OK;
}

int stage(int slot, size_t bytes, void** out) {
    if (bytes == 0) bytes = 4;
    if (g_ctx.stage_bytes[slot] < bytes) {
        if (g_ctx.stage[slot]) (void)hipFree(g_ctx.stage[slot]);
        g_ctx.stage[slot] = nullptr;
        g_ctx.stage_bytes[slot] = 0;
        size_t want = bytes + (bytes >> 2);
        if (hipMalloc(&g_ctx.stage[slot], want) != hipSuccess) {
            (void)hipGetLastError();
            return set_error(MXH_ERR_OOM, "staging allocation of %zu bytes failed", want);
        }
        g_ctx.stage_bytes[slot] = want;
    }
    *out = g_ctx.stage[slot];
    return MXH_OK;
}

// device copy of a host weight, uploading on first use
int device_weight(const void* host, size_t bytes, const void** dev) {
    auto key = std::make_pair(host, bytes);
    auto it = g_ctx.weights.find(key);
    if (it != g_ctx.weights.end()) {
        *dev = it->second;
        return MXH_OK;
    }
    void* d = nullptr;
    if (hipMalloc(&d, bytes + 256) != hipSuccess) {
        (void)hipGetLastError();
        return set_error(MXH_ERR_OOM, "weight upload: allocation of %zu bytes failed", bytes);
    }
    int rc = check_hip(hipMemcpy(d, host, bytes, hipMemcpyHostToDevice), "weight upload");
    if (rc) {
        (void)hipFree(d);
        return rc;
    }
    g_ctx.weights[key] = d;
    *dev = d;
    return MXH_OK;
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

int check_weight_ptr(int type, const void* w) {
    if (!w) return set_error(MXH_ERR_ARG, "null weight pointer");
    // blocks of 34, 22 and 210 bytes: 2-aligned blocks read through 4-aligned windows
    const size_t need = (type == MXH_Q8_0 || type == MXH_Q5_0 || type == MXH_Q6_K) ? 4 : 16;
    if (!aligned(w, need)) return set_error(MXH_ERR_ARG, "weight pointer must be %zu-byte aligned", need);
    return MXH_OK;
}

}  // namespace

int set_error(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int check_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return MXH_OK;
    return set_error(MXH_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

hipStream_t lib_stream() { return g_ctx.stream; }

}  // namespace mxh

using namespace mxh;

extern "C" {

int mxh_init(int device) {
    if (g_ctx.ready) return device == g_ctx.device ? MXH_OK : set_error(MXH_ERR_ARG, "already bound to device %d", g_ctx.device);
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        return set_error(MXH_ERR_NODEV, "no HIP device visible");
    }
    if (device < 0 || device >= n) return set_error(MXH_ERR_ARG, "device %d out of range (%d visible)", device, n);
    hipDeviceProp_t prop;
    if (int rc = check_hip(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties")) return rc;
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return set_error(MXH_ERR_NODEV, "device %d is %s; this library is built for gfx950", device, prop.gcnArchName);
    if (device >= kMaxDevices) return set_error(MXH_ERR_ARG, "device %d beyond the %d the library tracks", device, kMaxDevices);
    if (int rc = check_hip(hipSetDevice(device), "hipSetDevice")) return rc;
    // the no-allocation entry's scratch on this device (now current)
    void* sp = nullptr;
    if (int rc = check_hip(hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)")) return rc;
    g_scratch_ptr[device] = sp;
    if (int rc = check_hip(hipStreamCreateWithFlags(&g_ctx.stream, hipStreamNonBlocking), "hipStreamCreate")) return rc;
    if (int rc = check_hip(hipEventCreate(&g_ctx.ev0), "hipEventCreate")) return rc;
    if (int rc = check_hip(hipEventCreate(&g_ctx.ev1), "hipEventCreate")) return rc;
    g_ctx.device = device;
    g_ctx.ready = true;
    return MXH_OK;
}

int mxh_is_available(void) { return ensure_ready() == MXH_OK ? 1 : 0; }

const char* mxh_last_error(void) { return g_err.c_str(); }

int mxh_synchronize(void) {
    if (int rc = ensure_ready()) return rc;
    return check_hip(hipStreamSynchronize(g_ctx.stream), "hipStreamSynchronize");
}

void* mxh_stream(void) { return ensure_ready() == MXH_OK ? (void*)g_ctx.stream : nullptr; }

int mxh_alloc(void** dptr, size_t bytes) {
    if (!dptr) return set_error(MXH_ERR_ARG, "null output pointer");
    if (int rc = ensure_ready()) return rc;
    // 256 bytes of slack: tail loads of the last block never leave the allocation
    if (hipMalloc(dptr, bytes + 256) != hipSuccess) {
        (void)hipGetLastError();
        *dptr = nullptr;
        return set_error(MXH_ERR_OOM, "hipMalloc(%zu) failed", bytes);
    }
    return MXH_OK;
}

int mxh_free(void* dptr) {
    if (!dptr) return MXH_OK;
    return check_hip(hipFree(dptr), "hipFree");
}

int mxh_upload(void* dst, const void* src, size_t bytes) {
    if (int rc = ensure_ready()) return rc;
    if (int rc = check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_ctx.stream), "upload")) return rc;
    return check_hip(hipStreamSynchronize(g_ctx.stream), "upload sync");
}

int mxh_download(void* dst, const void* src, size_t bytes) {
    if (int rc = ensure_ready()) return rc;
    if (int rc = check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_ctx.stream), "download")) return rc;
    return check_hip(hipStreamSynchronize(g_ctx.stream), "download sync");
}

int mxh_memset(void* dptr, int value, size_t bytes) {
    if (int rc = ensure_ready()) return rc;
    return check_hip(hipMemsetAsync(dptr, value, bytes, g_ctx.stream), "memset");
}

int mxh_copy(void* dst, const void* src, size_t bytes) {
    if (int rc = ensure_ready()) return rc;
    if (!dst || !src) return set_error(MXH_ERR_ARG, "copy: null pointer");
    return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_ctx.stream), "copy");
}

int mxh_timer_begin(void) {
    if (int rc = ensure_ready()) return rc;
    return check_hip(hipEventRecord(g_ctx.ev0, g_ctx.stream), "hipEventRecord");
}

int mxh_timer_end(float* ms) {
    if (int rc = ensure_ready()) return rc;
    if (int rc = check_hip(hipEventRecord(g_ctx.ev1, g_ctx.stream), "hipEventRecord")) return rc;
    if (int rc = check_hip(hipEventSynchronize(g_ctx.ev1), "hipEventSynchronize")) return rc;
    return check_hip(hipEventElapsedTime(ms, g_ctx.ev0, g_ctx.ev1), "hipEventElapsedTime");
}

int mxh_gemv(int type, const void* w, const float* x, float* y, int64_t n, int64_t k, int form) {
    if (int rc = ensure_ready()) return rc;
    if (int rc = check_weight_ptr(type, w)) return rc;
    if (!x || !y || !aligned(x, 16)) return set_error(MXH_ERR_ARG, "x must be non-null and 16-byte aligned");
    if (type >= kTiledFlag && (type != (kTiledFlag | storage_type(type)) || tiled_type(storage_type(type), k) != type))
        return set_error(MXH_ERR_ARG, "gemv: type %d is not the tiled form of rows of %lld columns", type, (long long)k);
    if (n <= 0 || k <= 0 || row_bytes(type, k) == 0)
        return set_error(MXH_ERR_ARG, "gemv: k=%lld is not a whole number of type-%d blocks", (long long)k, type);
    int rc = gemv_launch(type, w, x, y, nullptr, n, k, form, g_ctx.stream);
    if (rc == MXH_ERR_ARG) return set_error(rc, "gemv: unsupported shape n=%lld k=%lld", (long long)n, (long long)k);
    if (rc == MXH_ERR_UNSUPPORTED) return set_error(rc, "gemv: unsupported type %d", type);
    return check_hip(hipGetLastError(), "gemv launch");
}

static_assert(MXH_TILED_FLAG == kTiledFlag, "public and internal tiled flags differ");

int mxh_tile_rows(int type, void* w, int64_t rows, int64_t cols, int* tiled) {
    if (int rc = ensure_ready()) return rc;
    if (!w || !tiled || rows <= 0 || cols <= 0 || type >= kTiledFlag || row_bytes(type, cols) == 0)
        return set_error(MXH_ERR_ARG, "tile_rows: bad arguments (type %d, %lld x %lld)", type, (long long)rows,
                         (long long)cols);
    if (!aligned(w, 16)) return set_error(MXH_ERR_ARG, "tile_rows: weight pointer must be 16-byte aligned");
    const int t = tiled_type(type, cols);
    if (t != type) {
        if (int rc = tile_rows_launch(type, w, rows, cols, g_ctx.stream)) return set_error(rc, "tile_rows: launch");
    }
    *tiled = t;
    return check_hip(hipGetLastError(), "tile_rows launch");
}

int mxh_matmul_rhs_t(int type, const float* a, int64_t m, const void* w, int64_t n, int64_t k, float* out, int form) {
    if (m <= 0) return set_error(MXH_ERR_ARG, "matmul: m must be positive");
    for (int64_t i = 0; i < m; ++i)
        if (int rc = mxh_gemv(type, w, a + i * k, out + i * n, n, k, form)) return rc;
    return MXH_OK;
}

int mxh_dequant(int type, const void* w, float* out, int64_t rows, int64_t cols, int form) {
    if (int rc = ensure_ready()) return rc;
    if (!w || !out) return set_error(MXH_ERR_ARG, "dequant: null pointer");
    int rc = dequant_launch(type, w, out, rows, cols, form, g_ctx.stream);
    if (rc) return set_error(rc, "dequant: bad type %d or shape %lldx%lld", type, (long long)rows, (long long)cols);
    return check_hip(hipGetLastError(), "dequant launch");
}

int mxh_gemm_q_bf16(int type, const float* a, int64_t m, const void* w, int64_t n, int64_t k, float* out, int form) {
    if (int rc = ensure_ready()) return rc;
    if (!a || !w || !out) return set_error(MXH_ERR_ARG, "gemm: null pointer");
    if (m <= 0 || n <= 0 || k <= 0 || k % 64 || m > INT32_MAX || n > INT32_MAX || k > INT32_MAX ||
        type >= kTiledFlag || row_bytes(type, k) == 0)
        return set_error(MXH_ERR_ARG, "gemm: bad shape %lldx%lldx%lld for type %d", (long long)m, (long long)n,
                         (long long)k, type);
    void* abf = nullptr;
    if (int rc = stage(3, (size_t)m * (size_t)k * 2, &abf)) return rc;
    if (int rc = rows_to_bf16_launch(a, (int)k, nullptr, 0.f, (int)k, (uint16_t*)abf, nullptr, (int)k, (int)m,
                                     g_ctx.stream))
        return set_error(rc, "gemm: conversion launch");
    if (int rc = gemm_bf16_run(type, (const uint16_t*)abf, nullptr, (int)k, w, out, (int)n, nullptr, (int)m, (int)n,
                               (int)k, form, nullptr, 0, g_ctx.stream))
        return set_error(rc, "gemm: unsupported type %d", type);
    return check_hip(hipGetLastError(), "gemm launch");
}


int mxh_gemm_q_f16(int type, const float* a, int64_t m, const void* w, int64_t n, int64_t k, float* out, int form) {
    if (int rc = ensure_ready()) return rc;
    if (int rc = gemm_q_f16_check("gemm_f16", type, a, m, w, n, k, out)) return rc;
    void* buf = nullptr;
    if (int rc = stage(2, f16_rows_bytes((size_t)m, (size_t)k), &buf)) return rc;
    return gemm_q_f16_body("gemm_f16", type, a, m, w, n, k, out, form, buf);
}

int mxh_gemm_q_f16_noalloc(int type, const float* a, int64_t m, const void* w, int64_t n, int64_t k, float* out,
                           int form) {
    if (int rc = ensure_ready()) return rc;
    if (int rc = gemm_q_f16_check("gemm_f16_noalloc", type, a, m, w, n, k, out)) return rc;
    if (f16_rows_bytes((size_t)m, (size_t)k) > kNoallocScratchBytes)
        return set_error(MXH_ERR_ARG, "gemm_f16_noalloc: %lld x %lld activations need %zu bytes of staging, above the "
                         "%zu-byte device scratch", (long long)m, (long long)k, f16_rows_bytes((size_t)m, (size_t)k),
                         kNoallocScratchBytes);
    void* buf = g_scratch_ptr[g_ctx.device];
    if (!buf) return set_error(MXH_ERR_HIP, "gemm_f16_noalloc: no scratch address for device %d", g_ctx.device);
    return gemm_q_f16_body("gemm_f16_noalloc", type, a, m, w, n, k, out, form, buf);
}

int mxh_attention_prefill(const float* q, const void* kc, const void* vc, float* att, int p0, int m, int nh, int nkv,
                          int hd) {
    if (int rc = ensure_ready()) return rc;
    if (!q || !kc || !vc || !att) return set_error(MXH_ERR_ARG, "attention_prefill: null pointer");
    if (m <= 0 || p0 < 0 || !attention_supported(nh, nkv, hd))
        return set_error(MXH_ERR_ARG, "attention_prefill: unsupported m %d p0 %d nh %d nkv %d hd %d", m, p0, nh, nkv,
                         hd);
    if (int rc = attention_rows_mfma_launch(q, (const __half*)kc, (const __half*)vc, att, p0, m, nh, nkv, hd,
                                            1.0f / sqrtf((float)hd), g_ctx.stream))
        return set_error(rc, "attention_prefill: launch");
    return check_hip(hipGetLastError(), "attention_prefill launch");
}

int mxh_sample(const float* logits, int n, int top_k, double temperature, double top_p, double min_p, uint64_t seed,
               uint64_t draw, int* token) {
    if (int rc = ensure_ready()) return rc;
    if (!logits || !token || n <= 0) return set_error(MXH_ERR_ARG, "sample: bad arguments");
    if (top_k < 1 || top_k > kSampleTopKMax || top_k > n)
        return set_error(MXH_ERR_ARG, "sample: top_k %d outside 1..min(%d, n)", top_k, kSampleTopKMax);
    void *prm = nullptr, *cand = nullptr;
    if (int rc = stage(0, sizeof(SampleParams) + sizeof(int), &prm)) return rc;
    if (int rc = stage(1, sample_scratch_keys(n, top_k) * sizeof(uint64_t), &cand)) return rc;
    SampleParams h{};
    h.top_k = top_k;
    h.temperature = temperature;
    h.top_p = top_p;
    h.min_p = min_p;
    h.seed = seed;
    h.draws = draw;
    int* out = reinterpret_cast<int*>(static_cast<char*>(prm) + sizeof(SampleParams));
    if (int rc = check_hip(hipMemcpyAsync(prm, &h, sizeof(h), hipMemcpyHostToDevice, g_ctx.stream), "sample params"))
        return rc;
    if (int rc = sample_launch(logits, n, static_cast<SampleParams*>(prm), top_k, static_cast<uint64_t*>(cand), out,
                               nullptr, nullptr, g_ctx.stream))
        return set_error(rc, "sample: vocabulary of %d too large for top_k %d", n, top_k);
    if (int rc = check_hip(hipMemcpyAsync(token, out, sizeof(int), hipMemcpyDeviceToHost, g_ctx.stream), "sample id"))
        return rc;
    return check_hip(hipStreamSynchronize(g_ctx.stream), "sample");
}

int mxh_preload(const void* host, size_t bytes) {
    if (int rc = ensure_ready()) return rc;
    if (!host || !bytes) return set_error(MXH_ERR_ARG, "preload: empty tensor");
    const void* d = nullptr;
    return device_weight(host, bytes, &d);
}

void mxh_release_resources(void) {
    if (!g_ctx.ready) return;
    (void)hipStreamSynchronize(g_ctx.stream);
    for (auto& kv : g_ctx.weights) (void)hipFree(kv.second);
    g_ctx.weights.clear();
    for (int i = 0; i < 4; ++i) {
        if (g_ctx.stage[i]) (void)hipFree(g_ctx.stage[i]);
        g_ctx.stage[i] = nullptr;
        g_ctx.stage_bytes[i] = 0;
    }
}

int mxh_host_matmul_rhs_t(int type, const float* a, int64_t m, int64_t k, const void* w, size_t w_bytes, int64_t n,
                          float* out, int form) {
    if (int rc = ensure_ready()) return rc;
    if (!a || !w || !out || m <= 0 || n <= 0 || k <= 0) return set_error(MXH_ERR_ARG, "matmul_rhs_t: bad arguments");
    const size_t rb = type >= kTiledFlag ? 0 : row_bytes(type, k);
    if (!rb || w_bytes < rb * (size_t)n) return set_error(MXH_ERR_ARG, "matmul_rhs_t: weight bytes too small");
    const void* dw = nullptr;
    if (int rc = device_weight(w, w_bytes, &dw)) return rc;  // the key mxh_preload(w, w_bytes) uses
    void *da = nullptr, *dout = nullptr;
    if (int rc = stage(0, sizeof(float) * (size_t)(m * k), &da)) return rc;
    if (int rc = stage(1, sizeof(float) * (size_t)(m * n), &dout)) return rc;
    if (int rc = check_hip(hipMemcpyAsync(da, a, sizeof(float) * m * k, hipMemcpyHostToDevice, g_ctx.stream), "H2D"))
        return rc;
    if (int rc = mxh_matmul_rhs_t(type, (const float*)da, m, dw, n, k, (float*)dout, form)) return rc;
    if (int rc = check_hip(hipMemcpyAsync(out, dout, sizeof(float) * m * n, hipMemcpyDeviceToHost, g_ctx.stream), "D2H"))
        return rc;
    return check_hip(hipStreamSynchronize(g_ctx.stream), "sync");
}

int mxh_host_matmul_f32(const float* a, const float* b, float* out, int64_t m, int64_t k, int64_t n) {
    if (int rc = ensure_ready()) return rc;
    if (!a || !b || !out || m <= 0 || k <= 0 || n <= 0) return set_error(MXH_ERR_ARG, "matmul: bad arguments");
    void *da, *db, *dout;
    if (int rc = stage(0, sizeof(float) * m * k, &da)) return rc;
    if (int rc = stage(2, sizeof(float) * k * n, &db)) return rc;
    if (int rc = stage(1, sizeof(float) * m * n, &dout)) return rc;
    if (int rc = check_hip(hipMemcpyAsync(da, a, sizeof(float) * m * k, hipMemcpyHostToDevice, g_ctx.stream), "copy")) return rc;
    if (int rc = check_hip(hipMemcpyAsync(db, b, sizeof(float) * k * n, hipMemcpyHostToDevice, g_ctx.stream), "copy")) return rc;
    int rc = matmul_f32_launch((const float*)da, (const float*)db, (float*)dout, m, k, n, g_ctx.stream);
    if (rc) return set_error(rc, "matmul: unsupported shape");
    if (int rc = check_hip(hipMemcpyAsync(out, dout, sizeof(float) * m * n, hipMemcpyDeviceToHost, g_ctx.stream), "copy")) return rc;
    return check_hip(hipStreamSynchronize(g_ctx.stream), "matmul");
}

int mxh_host_matmul_q(int type, const float* a, int64_t m, int64_t k, const void* b, size_t b_bytes, int64_t n,
                      float* out, int form) {
    if (int rc = ensure_ready()) return rc;
    if (!a || !b || !out || m <= 0 || k <= 0 || n <= 0) return set_error(MXH_ERR_ARG, "matmul: bad arguments");
    if (type == MXH_F32) {
        if (b_bytes < sizeof(float) * (size_t)k * (size_t)n) return set_error(MXH_ERR_ARG, "matmul: B too small");
        return mxh_host_matmul_f32(a, static_cast<const float*>(b), out, m, k, n);
    }
    const size_t rb = type >= kTiledFlag ? 0 : row_bytes(type, n);
    if (!rb) return set_error(MXH_ERR_ARG, "matmul: n=%lld is not a whole number of type-%d blocks", (long long)n, type);
    if (b_bytes < rb * (size_t)k) return set_error(MXH_ERR_ARG, "matmul: B holds %zu bytes, %zu needed", b_bytes, rb * (size_t)k);
    const void* db = nullptr;
    if (int rc = device_weight(b, b_bytes, &db)) return rc;
    void *da = nullptr, *dbf = nullptr, *dout = nullptr;
    if (int rc = stage(0, sizeof(float) * (size_t)(m * k), &da)) return rc;
    if (int rc = stage(2, sizeof(float) * (size_t)(k * n), &dbf)) return rc;
    if (int rc = stage(1, sizeof(float) * (size_t)(m * n), &dout)) return rc;
    if (int rc = check_hip(hipMemcpyAsync(da, a, sizeof(float) * m * k, hipMemcpyHostToDevice, g_ctx.stream), "copy")) return rc;
    if (int rc = dequant_launch(type, db, (float*)dbf, k, n, form, g_ctx.stream))
        return set_error(rc, "matmul: type %d with rows of %lld columns is not supported", type, (long long)n);
    if (int rc = matmul_f32_launch((const float*)da, (const float*)dbf, (float*)dout, m, k, n, g_ctx.stream))
        return set_error(rc, "matmul: unsupported shape");
    if (int rc = check_hip(hipMemcpyAsync(out, dout, sizeof(float) * m * n, hipMemcpyDeviceToHost, g_ctx.stream), "copy")) return rc;
    return check_hip(hipStreamSynchronize(g_ctx.stream), "matmul");
}

int mxh_host_vec_mul_rows_cols(const float* vec, const float* rows, float* out, size_t nrows, size_t ncols,
                               size_t stride) {
    if (int rc = ensure_ready()) return rc;
    // any stride is accepted, as in cpu_backend.cpp:379-393 (rows may overlap)
    if (!vec || !rows || !out || !nrows || !ncols) return set_error(MXH_ERR_ARG, "vec_mul_rows_cols: bad arguments");
    const size_t span = (nrows - 1) * stride + ncols;
    void *dv, *dr, *dout;
    if (int rc = stage(0, sizeof(float) * nrows, &dv)) return rc;
    if (int rc = stage(2, sizeof(float) * span, &dr)) return rc;
    if (int rc = stage(1, sizeof(float) * ncols, &dout)) return rc;
    if (int rc = check_hip(hipMemcpyAsync(dv, vec, sizeof(float) * nrows, hipMemcpyHostToDevice, g_ctx.stream), "copy")) return rc;
    if (int rc = check_hip(hipMemcpyAsync(dr, rows, sizeof(float) * span, hipMemcpyHostToDevice, g_ctx.stream), "copy")) return rc;
    if (int rc = vec_mul_rows_cols_launch((const float*)dv, (const float*)dr, (float*)dout, (int64_t)nrows,
                                          (int64_t)ncols, (int64_t)stride, g_ctx.stream))
        return set_error(rc, "vec_mul_rows_cols: bad shape");
    if (int rc = check_hip(hipMemcpyAsync(out, dout, sizeof(float) * ncols, hipMemcpyDeviceToHost, g_ctx.stream), "copy")) return rc;
    return check_hip(hipStreamSynchronize(g_ctx.stream), "vec_mul_rows_cols");
}

int mxh_host_matvec_strided(const float* vec, const float* mat, float* out, size_t K, size_t N, size_t stride) {
    // out[n] = sum_k vec[k] * mat[k*stride + n]: the same contraction as
    // vec_mul_rows_cols with K rows of N columns
    return mxh_host_vec_mul_rows_cols(vec, mat, out, K, N, stride);
}

int mxh_host_vec_dot_rows_ring(const float* vec, const float* ring, size_t head, size_t seq_max, size_t len, size_t K,
                               size_t stride, float* out) {
    if (int rc = ensure_ready()) return rc;
    // cpu_backend.cpp:364-377 accepts any stride and len > seq_max (the ring
    // is walked again); so does the kernel
    if (!vec || !ring || !out || !K || !len || !seq_max)
        return set_error(MXH_ERR_ARG, "vec_dot_rows_ring: bad arguments");
    const size_t span = (seq_max - 1) * stride + K;
    void *dv, *dr, *dout;
    if (int rc = stage(0, sizeof(float) * K, &dv)) return rc;
    if (int rc = stage(2, sizeof(float) * span, &dr)) return rc;
    if (int rc = stage(1, sizeof(float) * len, &dout)) return rc;
    if (int rc = check_hip(hipMemcpyAsync(dv, vec, sizeof(float) * K, hipMemcpyHostToDevice, g_ctx.stream), "copy")) return rc;
    if (int rc = check_hip(hipMemcpyAsync(dr, ring, sizeof(float) * span, hipMemcpyHostToDevice, g_ctx.stream), "copy")) return rc;
    if (int rc = vec_dot_rows_launch((const float*)dv, (const float*)dr, (float*)dout, (int64_t)K, (int64_t)len,
                                     (int64_t)stride, (int64_t)(head % seq_max), (int64_t)seq_max, g_ctx.stream))
        return set_error(rc, "vec_dot_rows: bad shape");
    if (int rc = check_hip(hipMemcpyAsync(out, dout, sizeof(float) * len, hipMemcpyDeviceToHost, g_ctx.stream), "copy")) return rc;
    return check_hip(hipStreamSynchronize(g_ctx.stream), "vec_dot_rows_ring");
}

int mxh_host_vec_dot_rows(const float* vec, const float* rows, float* out, size_t K, size_t nrows, size_t stride) {
    if (!nrows) return set_error(MXH_ERR_ARG, "vec_dot_rows: no rows");
    // contiguous rows are a ring that never wraps
    return mxh_host_vec_dot_rows_ring(vec, rows, 0, nrows, nrows, K, stride, out);
}

}  // extern "C"
