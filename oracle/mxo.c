/*
 * mxo.c — CPU oracle (TEST INFRASTRUCTURE ONLY; see mxo.h).
 *
 * Restates the reference CPU arithmetic.  Reference citations are relative
 * to the minXfmr.cpp source tree.
 */
#define _GNU_SOURCE
#include "mxo.h"

#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <limits.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* fp16                                                                */
/* ------------------------------------------------------------------ */

/* IEEE binary16 -> binary32, subnormals normalised (tensor.cpp:366-393). */
float mxo_fp16_to_fp32(uint16_t h)
{
    uint32_t s = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 31u;
    uint32_t f = h & 1023u;
    uint32_t bits;
    if (e == 31u) {
        bits = s | 0x7f800000u | (f << 13);
    } else if (e != 0u) {
        bits = s | ((e + 112u) << 23) | (f << 13);
    } else if (f == 0u) {
        bits = s;
    } else {
        /* subnormal: value = f * 2^-24; renormalise the mantissa */
        int shift = 0;
        while (!(f & 1024u)) { f <<= 1; ++shift; }
        bits = s | ((uint32_t)(113 - shift) << 23) | ((f & 1023u) << 13);
    }
    float v;
    memcpy(&v, &bits, 4);
    return v;
}

/* binary32 -> binary16, round to nearest even (used to model the fp16 KV
 * cache and to store quantizer scales; tensor.cpp:496-530 is the reference's
 * own encoder for its packed transpose). */
uint16_t mxo_fp32_to_fp16(float v)
{
    uint32_t x;
    memcpy(&x, &v, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {               /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    }
    if (ax >= 0x477ff000u) {               /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (ax < 0x38800000u) {                /* result subnormal or zero */
        if (ax < 0x33000000u) return (uint16_t)sign;  /* < 2^-25 -> 0 */
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        int e = (int)(ax >> 23);           /* biased, 102..112 */
        int sh = 126 - e;                  /* 14..24 */
        uint32_t q = m >> sh;
        uint32_t rem = m & ((1u << sh) - 1u);
        uint32_t half = 1u << (sh - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (ax >> 23) - 112u;
    uint32_t m = ax & 0x7fffffu;
    uint32_t r = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return (uint16_t)(sign | r);
}

/* ------------------------------------------------------------------ */
/* block formats                                                       */
/* ------------------------------------------------------------------ */

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* 6-bit (scale, min) of sub-block j from the 12-byte packed field.
 * j < 4: low six bits of bytes j and j+4 (tensor.cpp:397-399).
 * j >= 4: low/high nibble of byte j+4 plus two top bits taken from byte j
 * for both values in the reference CPU form (tensor.cpp:400-402); the ggml
 * form takes the scale's top bits from byte j-4 (cuda_backend.cu:175-183,
 * backend_runtime.cpp:76-84). */
void mxo_scale_min_k4(int j, const uint8_t *q, int form, uint8_t *sc, uint8_t *mn)
{
    if (j < 4) {
        *sc = q[j] & 0x3f;
        *mn = q[j + 4] & 0x3f;
        return;
    }
    const uint8_t lo = q[j + 4];
    const uint8_t top_sc = (uint8_t)((form == MXO_FORM_GGML ? q[j - 4] : q[j]) >> 6);
    const uint8_t top_mn = (uint8_t)(q[j] >> 6);
    *sc = (uint8_t)((lo & 0x0f) | (top_sc << 4));
    *mn = (uint8_t)((lo >> 4) | (top_mn << 4));
}

/* Q4_K: d@0, dmin@2, scales@4 (12 B), qs@16 (128 B).  Element
 * 64g + i (i < 32) is the low nibble of qs[32g + i]; 64g + 32 + i is its
 * high nibble; value = (d*sc)*q - (dmin*m) (tensor.cpp:405-432). */
void mxo_dequant_q4k_block(const uint8_t *blk, float *y, int form)
{
    const float d = mxo_fp16_to_fp32(rd16(blk));
    const float dmin = mxo_fp16_to_fp32(rd16(blk + 2));
    const uint8_t *scales = blk + 4;
    const uint8_t *qs = blk + 16;
    for (int g = 0; g < 4; ++g) {
        uint8_t sa, ma, sb, mb;
        mxo_scale_min_k4(2 * g, scales, form, &sa, &ma);
        mxo_scale_min_k4(2 * g + 1, scales, form, &sb, &mb);
        const float da = d * (float)sa, mma = dmin * (float)ma;
        const float db = d * (float)sb, mmb = dmin * (float)mb;
        const uint8_t *q = qs + 32 * g;
        for (int i = 0; i < 32; ++i) {
            y[64 * g + i] = da * (float)(q[i] & 0x0f) - mma;
            y[64 * g + 32 + i] = db * (float)(q[i] >> 4) - mmb;
        }
    }
}

/* Q5_K (absent from the reference, gguf_reader.cpp:1102-1115 rejects it).
 * Published ggml layout: d@0, dmin@2, scales@4 (12 B, Q4_K packing),
 * qh@16 (32 B), qs@48 (128 B); the fifth bit of element 64g+i is bit 2g of
 * qh[i], of element 64g+32+i bit 2g+1.  The same scale-form switch applies. */
void mxo_dequant_q5k_block(const uint8_t *blk, float *y, int form)
{
    const float d = mxo_fp16_to_fp32(rd16(blk));
    const float dmin = mxo_fp16_to_fp32(rd16(blk + 2));
    const uint8_t *scales = blk + 4;
    const uint8_t *qh = blk + 16;
    const uint8_t *qs = blk + 48;
    for (int g = 0; g < 4; ++g) {
        uint8_t sa, ma, sb, mb;
        mxo_scale_min_k4(2 * g, scales, form, &sa, &ma);
        mxo_scale_min_k4(2 * g + 1, scales, form, &sb, &mb);
        const float da = d * (float)sa, mma = dmin * (float)ma;
        const float db = d * (float)sb, mmb = dmin * (float)mb;
        const uint8_t *q = qs + 32 * g;
        for (int i = 0; i < 32; ++i) {
            const int lo = (q[i] & 0x0f) | (((qh[i] >> (2 * g)) & 1) << 4);
            const int hi = (q[i] >> 4) | (((qh[i] >> (2 * g + 1)) & 1) << 4);
            y[64 * g + i] = da * (float)lo - mma;
            y[64 * g + 32 + i] = db * (float)hi - mmb;
        }
    }
}

/* Q8_0: d@0 (fp16), 32 x int8; value = d*q (tensor.cpp:451-457). */
void mxo_dequant_q8_0_block(const uint8_t *blk, float *y)
{
    const float d = mxo_fp16_to_fp32(rd16(blk));
    const int8_t *q = (const int8_t *)(blk + 2);
    for (int i = 0; i < 32; ++i) y[i] = d * (float)q[i];
}

/* Q5_0: d@0, qh@2 (32-bit mask), qs@6; element i (i<16) = low nibble of
 * qs[i] | bit i of qh << 4, element 16+i = high nibble | bit 16+i << 4;
 * value = d*(q-16) (tensor.cpp:434-449). */
void mxo_dequant_q5_0_block(const uint8_t *blk, float *y)
{
    const float d = mxo_fp16_to_fp32(rd16(blk));
    const uint32_t qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) | ((uint32_t)blk[4] << 16) |
                        ((uint32_t)blk[5] << 24);
    const uint8_t *qs = blk + 6;
    for (int i = 0; i < 16; ++i) {
        const int a = (qs[i] & 0x0f) | (int)(((qh >> i) & 1u) << 4);
        const int b = (qs[i] >> 4) | (int)(((qh >> (i + 16)) & 1u) << 4);
        y[i] = d * (float)(a - 16);
        y[i + 16] = d * (float)(b - 16);
    }
}

/* Q6_K (GGML type 14), which the reference converts to F32 at load
 * (gguf_reader.cpp:905-1008): ql@0 (128 B), qh@128 (64 B), scales@192
 * (16 x int8), d@208 (fp16).  Half h (elements 128h..128h+127) reads
 * ql[64h..], qh[32h..], scales[8h..]; for l < 32 its elements l, l+32,
 * l+64, l+96 take the low nibble of ql[l], the low nibble of ql[l+32], the
 * high nibble of ql[l], the high nibble of ql[l+32], each with the 2-bit
 * field 0, 1, 2, 3 of qh[l] above it, minus 32; element e scales by
 * scales[e / 16].  value = (d * sc) * q, in that float order. */
void mxo_dequant_q6k_block(const uint8_t *blk, float *y)
{
    const uint8_t *ql = blk, *qh = blk + 128;
    const int8_t *sc = (const int8_t *)(blk + 192);
    const float d = mxo_fp16_to_fp32(rd16(blk + 208));
    for (int h = 0; h < 2; ++h) {
        for (int l = 0; l < 32; ++l) {
            const uint8_t a = ql[64 * h + l], b = ql[64 * h + 32 + l], c = qh[32 * h + l];
            const int q0 = (int)((a & 15u) | ((c & 3u) << 4)) - 32;
            const int q1 = (int)((b & 15u) | (((c >> 2) & 3u) << 4)) - 32;
            const int q2 = (int)((a >> 4) | (((c >> 4) & 3u) << 4)) - 32;
            const int q3 = (int)((b >> 4) | (((c >> 6) & 3u) << 4)) - 32;
            const int e = 128 * h + l;
            y[e] = d * (float)sc[e >> 4] * (float)q0;
            y[e + 32] = d * (float)sc[(e + 32) >> 4] * (float)q1;
            y[e + 64] = d * (float)sc[(e + 64) >> 4] * (float)q2;
            y[e + 96] = d * (float)sc[(e + 96) >> 4] * (float)q3;
        }
    }
}

size_t mxo_block_elems(int type)
{
    switch (type) {
    case MXO_F32: case MXO_F16: case MXO_Q1_0: return 1;
    case MXO_Q5_0: case MXO_Q8_0: return 32;
    case MXO_Q4_K: case MXO_Q5_K: case MXO_Q6_K: return 256;
    }
    return 0;
}

size_t mxo_block_bytes(int type)
{
    switch (type) {
    case MXO_F32: return 4;
    case MXO_F16: return 2;
    case MXO_Q1_0: return 1;
    case MXO_Q5_0: return 22;
    case MXO_Q8_0: return 34;
    case MXO_Q4_K: return 144;
    case MXO_Q5_K: return 176;
    case MXO_Q6_K: return 210;
    }
    return 0;
}

/* tensor.cpp tensor_q*_row_bytes: 0 when cols is not a whole number of blocks */
size_t mxo_row_bytes(int type, size_t cols)
{
    const size_t be = mxo_block_elems(type);
    if (be == 0 || cols % be) return 0;
    return cols / be * mxo_block_bytes(type);
}

static void dequant_block(int type, const uint8_t *blk, float *y, int form)
{
    switch (type) {
    case MXO_Q4_K: mxo_dequant_q4k_block(blk, y, form); break;
    case MXO_Q5_K: mxo_dequant_q5k_block(blk, y, form); break;
    case MXO_Q8_0: mxo_dequant_q8_0_block(blk, y); break;
    case MXO_Q5_0: mxo_dequant_q5_0_block(blk, y); break;
    case MXO_Q6_K: mxo_dequant_q6k_block(blk, y); break;
    case MXO_F32: memcpy(y, blk, 4); break;
    case MXO_F16: y[0] = mxo_fp16_to_fp32(rd16(blk)); break;
    case MXO_Q1_0: y[0] = (float)blk[0]; break; /* gguf_reader.cpp:1038 */
    }
}

/* tensor_dequant_row over a row range (tensor.cpp:459-493). */
int mxo_dequant_rows(int type, const void *w, size_t rows, size_t cols, float *out, int form)
{
    const size_t rb = mxo_row_bytes(type, cols);
    if (!rb) return -1;
    const size_t be = mxo_block_elems(type), bb = mxo_block_bytes(type);
    for (size_t r = 0; r < rows; ++r) {
        const uint8_t *src = (const uint8_t *)w + r * rb;
        for (size_t b = 0; b < cols / be; ++b) dequant_block(type, src + b * bb, out + r * cols + b * be, form);
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* rhs-transposed matmul (the decode hot op)                           */
/* ------------------------------------------------------------------ */

/* Per-block dot products with the reference accumulation types:
 *  Q4_K: dequantize the 256-element block to float, sum x*w in double,
 *        return float (backend_runtime.cpp:86-95).  Q5_K follows Q4_K.
 *  Q8_0: float accumulator, acc += x*(d*q) (backend_runtime.cpp:126-137).
 *  Q5_0: float accumulator, same pattern (backend_runtime.cpp:97-124).
 * The reference is built with -O3 -march=native under gnu++17, whose
 * default -ffp-contract=fast turns the float update into a fused
 * multiply-add; fmaf() states that explicitly. */
static float dot_block(int type, const uint8_t *blk, const float *x, int form)
{
    if (type == MXO_Q4_K || type == MXO_Q5_K) {
        float w[256];
        if (type == MXO_Q4_K) mxo_dequant_q4k_block(blk, w, form);
        else mxo_dequant_q5k_block(blk, w, form);
        double acc = 0.0;
        for (int i = 0; i < 256; ++i) acc += (double)w[i] * (double)x[i];
        return (float)acc;
    }
    if (type == MXO_Q8_0) {
        const float d = mxo_fp16_to_fp32(rd16(blk));
        const int8_t *q = (const int8_t *)(blk + 2);
        float acc = 0.0f;
        for (int i = 0; i < 32; ++i) acc = fmaf(x[i], d * (float)q[i], acc);
        return acc;
    }
    if (type == MXO_Q5_0) {
        float w[32];
        mxo_dequant_q5_0_block(blk, w);
        float acc = 0.0f;
        for (int i = 0; i < 16; ++i) {
            acc = fmaf(x[i], w[i], acc);
            acc = fmaf(x[i + 16], w[i + 16], acc);
        }
        return acc;
    }
    return 0.0f;
}

/* backend_runtime.cpp:266-376: out[i][j] = float sum over blocks (in block
 * order) of the per-block dot.  F32 weights are read as [N x K] rows, which
 * is the reference CUDA kernel's reading (cuda_backend.cu:731-747); the
 * reference CPU F32 branch indexes B as [K x N] (backend_runtime.cpp:425),
 * an inconsistency no GGUF projection in the benchmark configs reaches. */
int mxo_matmul_rhs_t(int type, const float *A, size_t M, size_t K, const void *B, size_t N,
                     float *out, int form, int nthreads)
{
    if (!A || !B || !out) return -1;
    if (type == MXO_F16 || type == MXO_Q6_K || type == MXO_Q1_0) {
        /* the reference converts F16, Q6_K and type-41 weights to F32 when
         * it loads them (gguf_reader.cpp:759-785, :905-1008, :1010-1098) and
         * multiplies the F32 values: each row is decoded, then summed as an
         * F32 row below */
        const size_t rb = mxo_row_bytes(type, K);
        if (!rb) return -1;
#pragma omp parallel for num_threads(nthreads > 0 ? nthreads : 1) schedule(static)
        for (long long j = 0; j < (long long)N; ++j) {
            float *w = (float *)malloc(K * sizeof(float));
            mxo_dequant_rows(type, (const uint8_t *)B + (size_t)j * rb, 1, K, w, form);
            for (size_t i = 0; i < M; ++i) {
                float s = 0.0f;
                for (size_t k = 0; k < K; ++k) s = fmaf(A[i * K + k], w[k], s);
                out[i * N + (size_t)j] = s;
            }
            free(w);
        }
        return 0;
    }
    if (type == MXO_F32) {
        const float *W = (const float *)B;
        long long work = (long long)(M * N);
#pragma omp parallel for num_threads(nthreads > 0 ? nthreads : 1) schedule(static)
        for (long long idx = 0; idx < work; ++idx) {
            const size_t i = (size_t)idx / N, j = (size_t)idx % N;
            float s = 0.0f;
            for (size_t k = 0; k < K; ++k) s = fmaf(A[i * K + k], W[j * K + k], s);
            out[i * N + j] = s;
        }
        return 0;
    }
    const size_t rb = mxo_row_bytes(type, K);
    if (!rb) return -1;
    const size_t be = mxo_block_elems(type), bb = mxo_block_bytes(type), nb = K / be;
    const long long work = (long long)(M * N);
#pragma omp parallel for num_threads(nthreads > 0 ? nthreads : 1) schedule(static)
    for (long long idx = 0; idx < work; ++idx) {
        const size_t i = (size_t)idx / N, j = (size_t)idx % N;
        const uint8_t *row = (const uint8_t *)B + j * rb;
        float s = 0.0f;
        for (size_t b = 0; b < nb; ++b) s += dot_block(type, row + b * bb, A + i * K + b * be, form);
        out[i * N + j] = s;
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* quantizers (synthetic-model generators; not part of the reference)   */
/* ------------------------------------------------------------------ */

static int iround(float v) { return (int)lrintf(v); }
static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

void mxo_quantize_q8_0_row(const float *x, size_t n, uint8_t *out)
{
    for (size_t b = 0; b < n / 32; ++b) {
        const float *v = x + 32 * b;
        uint8_t *o = out + 34 * b;
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
        const uint16_t dh = mxo_fp32_to_fp16(amax / 127.0f);
        const float d = mxo_fp16_to_fp32(dh);
        o[0] = (uint8_t)(dh & 0xff);
        o[1] = (uint8_t)(dh >> 8);
        for (int i = 0; i < 32; ++i) o[2 + i] = (uint8_t)(int8_t)(d > 0.0f ? clampi(iround(v[i] / d), -127, 127) : 0);
    }
}

void mxo_quantize_q5_0_row(const float *x, size_t n, uint8_t *out)
{
    for (size_t b = 0; b < n / 32; ++b) {
        const float *v = x + 32 * b;
        uint8_t *o = out + 22 * b;
        float amax = 0.0f, mx = 0.0f;
        for (int i = 0; i < 32; ++i) if (fabsf(v[i]) > amax) { amax = fabsf(v[i]); mx = v[i]; }
        const uint16_t dh = mxo_fp32_to_fp16(mx / -16.0f);
        const float d = mxo_fp16_to_fp32(dh);
        uint32_t qh = 0;
        memset(o + 6, 0, 16);
        for (int i = 0; i < 32; ++i) {
            const int q = d != 0.0f ? clampi(iround(v[i] / d) + 16, 0, 31) : 16;
            const int pos = i < 16 ? i : i - 16;
            o[6 + pos] |= (uint8_t)((q & 15) << (i < 16 ? 0 : 4));
            qh |= (uint32_t)(q >> 4) << i;
        }
        o[0] = (uint8_t)(dh & 0xff);
        o[1] = (uint8_t)(dh >> 8);
        o[2] = (uint8_t)qh; o[3] = (uint8_t)(qh >> 8); o[4] = (uint8_t)(qh >> 16); o[5] = (uint8_t)(qh >> 24);
    }
}

/* Q6_K: per 16-element sub-block a signed scale (amax / 31 over d, d the
 * largest such scale / 127), codes q + 32 in [0, 63], packed as
 * mxo_dequant_q6k_block reads them. */
void mxo_quantize_q6k_row(const float *x, size_t n, uint8_t *out)
{
    for (size_t b = 0; b < n / 256; ++b) {
        const float *v = x + 256 * b;
        uint8_t *o = out + 210 * b;
        float sf[16], smax = 0.0f;
        for (int j = 0; j < 16; ++j) {
            float amax = 0.0f;
            for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[16 * j + i]));
            sf[j] = amax / 31.0f;
            smax = fmaxf(smax, sf[j]);
        }
        const uint16_t dh = mxo_fp32_to_fp16(smax / 127.0f);
        const float d = mxo_fp16_to_fp32(dh);
        int q[256];
        for (int j = 0; j < 16; ++j) {
            const int sc = d > 0.0f ? clampi(iround(sf[j] / d), -128, 127) : 0;
            o[192 + j] = (uint8_t)(int8_t)sc;
            const float ds = d * (float)sc;
            for (int i = 0; i < 16; ++i)
                q[16 * j + i] = (ds != 0.0f ? clampi(iround(v[16 * j + i] / ds), -32, 31) : 0) + 32;
        }
        memset(o, 0, 192);
        for (int h = 0; h < 2; ++h)
            for (int l = 0; l < 32; ++l) {
                const int *qq = q + 128 * h + l;
                o[64 * h + l] = (uint8_t)((qq[0] & 15) | ((qq[64] & 15) << 4));
                o[64 * h + 32 + l] = (uint8_t)((qq[32] & 15) | ((qq[96] & 15) << 4));
                o[128 + 32 * h + l] =
                    (uint8_t)((qq[0] >> 4) | ((qq[32] >> 4) << 2) | ((qq[64] >> 4) << 4) | ((qq[96] >> 4) << 6));
            }
        o[208] = (uint8_t)dh;
        o[209] = (uint8_t)(dh >> 8);
    }
}

/* Pack 8 (scale, min) pairs of 6 bits each in the ggml K-quant layout. */
static void pack_scales_k4(const int *sc, const int *mn, uint8_t *s12)
{
    memset(s12, 0, 12);
    for (int j = 0; j < 8; ++j) {
        if (j < 4) {
            s12[j] = (uint8_t)sc[j];
            s12[j + 4] = (uint8_t)mn[j];
        } else {
            s12[j + 4] = (uint8_t)((sc[j] & 15) | ((mn[j] & 15) << 4));
            s12[j - 4] |= (uint8_t)((sc[j] >> 4) << 6);
            s12[j] |= (uint8_t)((mn[j] >> 4) << 6);
        }
    }
}

/* Affine min/max K-quant of one 256-block into nbits-bit codes: sub-block
 * scale = (max-min)/qmax, offset = -min (min clipped at 0), both requantized
 * to 6 bits against the block's fp16 d / dmin. */
static void quantize_k_block(const float *v, int qmax, uint16_t *dh_out, uint16_t *mh_out,
                             int *sc6, int *mn6, int *codes)
{
    float scale[8], offs[8];
    float smax = 0.0f, omax = 0.0f;
    for (int j = 0; j < 8; ++j) {
        float lo = v[32 * j], hi = v[32 * j];
        for (int i = 1; i < 32; ++i) { lo = fminf(lo, v[32 * j + i]); hi = fmaxf(hi, v[32 * j + i]); }
        if (lo > 0.0f) lo = 0.0f;
        scale[j] = (hi - lo) / (float)qmax;
        offs[j] = -lo;
        smax = fmaxf(smax, scale[j]);
        omax = fmaxf(omax, offs[j]);
    }
    const uint16_t dh = mxo_fp32_to_fp16(smax / 63.0f);
    const uint16_t mh = mxo_fp32_to_fp16(omax / 63.0f);
    const float d = mxo_fp16_to_fp32(dh), dm = mxo_fp16_to_fp32(mh);
    for (int j = 0; j < 8; ++j) {
        sc6[j] = d > 0.0f ? clampi(iround(scale[j] / d), 0, 63) : 0;
        mn6[j] = dm > 0.0f ? clampi(iround(offs[j] / dm), 0, 63) : 0;
        const float ds = d * (float)sc6[j], ms = dm * (float)mn6[j];
        for (int i = 0; i < 32; ++i)
            codes[32 * j + i] = ds > 0.0f ? clampi(iround((v[32 * j + i] + ms) / ds), 0, qmax) : 0;
    }
    *dh_out = dh;
    *mh_out = mh;
}

void mxo_quantize_q4k_row(const float *x, size_t n, uint8_t *out)
{
    for (size_t b = 0; b < n / 256; ++b) {
        uint8_t *o = out + 144 * b;
        int sc[8], mn[8], q[256];
        uint16_t dh, mh;
        quantize_k_block(x + 256 * b, 15, &dh, &mh, sc, mn, q);
        o[0] = (uint8_t)dh; o[1] = (uint8_t)(dh >> 8);
        o[2] = (uint8_t)mh; o[3] = (uint8_t)(mh >> 8);
        pack_scales_k4(sc, mn, o + 4);
        for (int g = 0; g < 4; ++g)
            for (int i = 0; i < 32; ++i)
                o[16 + 32 * g + i] = (uint8_t)(q[64 * g + i] | (q[64 * g + 32 + i] << 4));
    }
}

void mxo_quantize_q5k_row(const float *x, size_t n, uint8_t *out)
{
    for (size_t b = 0; b < n / 256; ++b) {
        uint8_t *o = out + 176 * b;
        int sc[8], mn[8], q[256];
        uint16_t dh, mh;
        quantize_k_block(x + 256 * b, 31, &dh, &mh, sc, mn, q);
        o[0] = (uint8_t)dh; o[1] = (uint8_t)(dh >> 8);
        o[2] = (uint8_t)mh; o[3] = (uint8_t)(mh >> 8);
        pack_scales_k4(sc, mn, o + 4);
        memset(o + 16, 0, 32);
        for (int g = 0; g < 4; ++g)
            for (int i = 0; i < 32; ++i) {
                const int a = q[64 * g + i], c = q[64 * g + 32 + i];
                o[48 + 32 * g + i] = (uint8_t)((a & 15) | ((c & 15) << 4));
                o[16 + i] |= (uint8_t)(((a >> 4) << (2 * g)) | ((c >> 4) << (2 * g + 1)));
            }
    }
}

/* ------------------------------------------------------------------ */
/* layer ops                                                           */
/* ------------------------------------------------------------------ */

/* rmsnorm_forward (rmsnorm.cpp:5-26): sum of squares in double,
 * y = float(x * (1/sqrt(mean + eps))), then the weight multiply in float
 * (apply_norm_scale, transformer.cpp:189-214). */
void mxo_rmsnorm(const float *x, const float *w, float *y, size_t n, float eps)
{
    double ss = 0.0;
    for (size_t i = 0; i < n; ++i) ss += (double)x[i] * (double)x[i];
    const double inv = 1.0 / sqrt(ss / (double)n + (double)eps);
    for (size_t i = 0; i < n; ++i) {
        float v = (float)((double)x[i] * inv);
        y[i] = w ? v * w[i] : v;
    }
}

/* rope_apply for one row (rope.cpp:6-57): inv_freq = 1/theta^(2i/rot),
 * cos/sin and the rotation in double, stored as float. */
void mxo_rope(float *v, size_t n_heads, size_t head_dim, size_t n_rot, size_t pos, float theta, int neox)
{
    size_t rot = n_rot ? n_rot : head_dim;
    if (rot > head_dim) rot = head_dim;
    rot &= ~(size_t)1;
    if (rot < 2) return;
    const size_t half = rot / 2;
    for (size_t i = 0; i < half; ++i) {
        const double inv_freq = 1.0 / pow((double)theta, (2.0 * (double)i) / (double)rot);
        const double ang = (double)pos * inv_freq;
        const double c = cos(ang), s = sin(ang);
        for (size_t h = 0; h < n_heads; ++h) {
            float *p = v + h * head_dim;
            const size_t a = neox ? i : 2 * i;
            const size_t b = neox ? i + half : 2 * i + 1;
            const double x0 = p[a], x1 = p[b];
            p[a] = (float)(x0 * c - x1 * s);
            p[b] = (float)(x0 * s + x1 * c);
        }
    }
}

/* softmax_row (softmax.cpp:4-18): float max, expf, double sum, float 1/sum. */
void mxo_softmax(float *row, size_t len)
{
    if (!len) return;
    float mx = row[0];
    for (size_t i = 1; i < len; ++i) if (row[i] > mx) mx = row[i];
    double sum = 0.0;
    for (size_t i = 0; i < len; ++i) { row[i] = expf(row[i] - mx); sum += row[i]; }
    if (sum <= 0.0) return;
    const float inv = (float)(1.0 / sum);
    for (size_t i = 0; i < len; ++i) row[i] *= inv;
}

/* silu_f32 (transformer.cpp:183-185) */
float mxo_silu(float x) { return x / (1.0f + expf(-x)); }

int mxo_argmax(const float *logits, size_t n)
{
    size_t best = 0;
    for (size_t i = 1; i < n; ++i) if (logits[i] > logits[best]) best = i;
    return (int)best;
}

/* splitmix64 -> uniform double in [0, 1) */
double mxo_rng_uniform(uint64_t *state)
{
    uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (double)(z >> 11) * (1.0 / 9007199254740992.0);
}

/* top-k candidates ordered by (logit desc, id asc); insertion into a small
 * sorted list keeps this O(n k). */
static int topk_select(const float *logits, size_t n, int k, int *ids)
{
    int cnt = 0;
    for (size_t i = 0; i < n; ++i) {
        const float v = logits[i];
        if (cnt == k && !(v > logits[ids[cnt - 1]])) continue;
        int p = cnt < k ? cnt++ : k - 1;
        while (p > 0 && v > logits[ids[p - 1]]) { ids[p] = ids[p - 1]; --p; }
        ids[p] = (int)i;
    }
    return cnt;
}

/* minxfmr.cpp:2091-2171 restated with a seeded uniform draw. */
int mxo_sample(const float *logits, size_t n, int top_k, double temperature, double top_p,
               double min_p, uint64_t *rng_state)
{
    if (top_k <= 0) top_k = 1;
    if ((size_t)top_k > n) top_k = (int)n;
    int *ids = (int *)malloc(sizeof(int) * (size_t)top_k);
    double *p = (double *)malloc(sizeof(double) * (size_t)top_k);
    const int k = topk_select(logits, n, top_k, ids);
    int pick = ids[0];
    if (temperature > 0.0) {
        if (top_p <= 0.0 || top_p > 1.0) top_p = 1.0;
        if (min_p < 0.0) min_p = 0.0;
        if (min_p > 1.0) min_p = 1.0;
        const double mx = logits[ids[0]];
        double sum = 0.0;
        for (int i = 0; i < k; ++i) { p[i] = exp(((double)logits[ids[i]] - mx) / temperature); sum += p[i]; }
        if (sum > 0.0) {
            for (int i = 0; i < k; ++i) p[i] /= sum;
            int m = k;
            if (top_p < 1.0) {
                double cum = 0.0;
                m = 0;
                for (int i = 0; i < k; ++i) { cum += p[i]; m = i + 1; if (cum >= top_p) break; }
                double r = 0.0;
                for (int i = 0; i < m; ++i) r += p[i];
                if (r > 0.0) for (int i = 0; i < m; ++i) p[i] /= r;
            }
            if (min_p > 0.0 && m > 1) {
                const double thr = p[0] * min_p;
                int keep = 1;
                for (int i = 1; i < m; ++i) { if (p[i] >= thr) keep = i + 1; else break; }
                m = keep;
                double r = 0.0;
                for (int i = 0; i < m; ++i) r += p[i];
                if (r > 0.0) for (int i = 0; i < m; ++i) p[i] /= r;
            }
            double total = 0.0;
            for (int i = 0; i < m; ++i) total += p[i];
            const double u = mxo_rng_uniform(rng_state) * total;
            double cum = 0.0;
            pick = ids[m - 1];
            for (int i = 0; i < m; ++i) { cum += p[i]; if (u < cum) { pick = ids[i]; break; } }
        }
    }
    free(ids);
    free(p);
    return pick;
}

/* minxfmr.cpp:2047-2089: suppressed ids to -inf, then the llama.cpp-style
 * penalties over the last repeat_last_n history ids (all when < 0), each
 * distinct id once with its count, in double.  The reference's logits are
 * doubles; here the edited value is rounded back to the float logits. */
void mxo_logit_edits(float *logits, size_t n, const int *history, size_t n_hist, const int *suppress,
                     size_t n_suppress, int repeat_last_n, double repeat_penalty, double frequency_penalty,
                     double presence_penalty)
{
    for (size_t j = 0; j < n_suppress; ++j)
        if (suppress[j] >= 0 && (size_t)suppress[j] < n) logits[suppress[j]] = -INFINITY;
    size_t pn = repeat_last_n < 0 ? n_hist : (size_t)repeat_last_n;
    if (pn > n_hist) pn = n_hist;
    if (pn == 0 || (repeat_penalty == 1.0 && frequency_penalty == 0.0 && presence_penalty == 0.0)) return;
    const int *win = history + (n_hist - pn);
    for (size_t i = 0; i < pn; ++i) {
        const int t = win[i];
        if (t < 0 || (size_t)t >= n) continue;
        int first = 1, count = 0;
        for (size_t j = 0; j < pn; ++j) {
            if (win[j] == t) {
                if (j < i) first = 0;
                ++count;
            }
        }
        if (!first) continue;
        double l = (double)logits[t];
        if (repeat_penalty != 1.0) l = l <= 0.0 ? l * repeat_penalty : l / repeat_penalty;
        l -= (double)count * frequency_penalty + (count > 0 ? presence_penalty : 0.0);
        logits[t] = (float)l;
    }
}

/* ------------------------------------------------------------------ */
/* GGUF reader (gguf_reader.cpp:224-676 semantics, exact names)        */
/* ------------------------------------------------------------------ */

typedef struct {
    char name[96];
    int type;
    uint64_t ne[4];
    int n_dims;
    uint64_t offset;
} gg_tensor;

typedef struct {
    const uint8_t *base;
    size_t size;
    size_t pos;
    int err;
} gg_cur;

static uint64_t gg_u(gg_cur *c, int nbytes)
{
    if (c->pos + (size_t)nbytes > c->size) { c->err = 1; return 0; }
    uint64_t v = 0;
    for (int i = 0; i < nbytes; ++i) v |= (uint64_t)c->base[c->pos + i] << (8 * i);
    c->pos += (size_t)nbytes;
    return v;
}

static void gg_str(gg_cur *c, char *dst, size_t cap)
{
    uint64_t len = gg_u(c, 8);
    if (c->err || c->pos + len > c->size) { c->err = 1; return; }
    if (dst) {
        size_t n = len < cap - 1 ? (size_t)len : cap - 1;
        memcpy(dst, c->base + c->pos, n);
        dst[n] = 0;
    }
    c->pos += (size_t)len;
}

static int gg_scalar_size(uint32_t t)
{
    switch (t) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
    }
    return -1;
}

typedef struct {
    int n_layer, n_embd, n_head, n_head_kv, n_ff, n_ctx_train, key_length;
    float eps, theta;
    int alignment;
} gg_hparams;

static double gg_read_num(gg_cur *c, uint32_t t)
{
    switch (t) {
    case 0: return (double)(uint8_t)gg_u(c, 1);
    case 1: return (double)(int8_t)gg_u(c, 1);
    case 2: return (double)(uint16_t)gg_u(c, 2);
    case 3: return (double)(int16_t)gg_u(c, 2);
    case 4: return (double)(uint32_t)gg_u(c, 4);
    case 5: return (double)(int32_t)gg_u(c, 4);
    case 6: { uint32_t b = (uint32_t)gg_u(c, 4); float f; memcpy(&f, &b, 4); return f; }
    case 7: return (double)gg_u(c, 1);
    case 10: return (double)gg_u(c, 8);
    case 11: return (double)(int64_t)gg_u(c, 8);
    case 12: { uint64_t b = gg_u(c, 8); double f; memcpy(&f, &b, 8); return f; }
    }
    c->err = 1;
    return 0;
}

static int ends_with(const char *s, const char *suf)
{
    size_t a = strlen(s), b = strlen(suf);
    return a >= b && strcmp(s + a - b, suf) == 0;
}

/* ------------------------------------------------------------------ */
/* model                                                               */
/* ------------------------------------------------------------------ */

typedef struct {
    int type;
    const uint8_t *data;
    size_t rows, cols;
} wt;

typedef struct {
    wt wq, wk, wv, wo, gate, up, down;
    const float *bq, *bk, *bv;
    const float *attn_norm, *ffn_norm, *q_norm, *k_norm;
} layer_w;

struct mxo_model {
    void *map;
    size_t map_size;
    gg_hparams hp;
    int n_vocab, head_dim, kv_dim, n_ctx;
    int flags, form, nthreads;
    layer_w *layers;
    wt embd, out;
    const float *out_norm;
    float *kcache, *vcache; /* [n_layer][n_ctx][kv_dim] */
    int pos;
    /* scratch */
    float *x, *xn, *q, *k, *v, *att, *o, *g, *u, *h, *scores;
};

static const gg_tensor *find_tensor(const gg_tensor *ts, uint64_t n, const char *name)
{
    for (uint64_t i = 0; i < n; ++i) if (strcmp(ts[i].name, name) == 0) return &ts[i];
    return NULL;
}

static int bind_w(const gg_tensor *ts, uint64_t n, const uint8_t *data0, const char *name, wt *w)
{
    const gg_tensor *t = find_tensor(ts, n, name);
    if (!t) return -1;
    w->type = t->type;
    w->cols = (size_t)t->ne[0];
    w->rows = t->n_dims > 1 ? (size_t)t->ne[1] : 1;
    w->data = data0 + t->offset;
    return 0;
}

static const float *bind_f32(const gg_tensor *ts, uint64_t n, const uint8_t *data0, const char *name)
{
    const gg_tensor *t = find_tensor(ts, n, name);
    if (!t || t->type != MXO_F32) return NULL;
    return (const float *)(data0 + t->offset);
}

mxo_model *mxo_model_open(const char *path, int n_ctx, int flags, int nthreads)
{
    int fd = open(path, O_RDONLY);
    if (fd < 0) return NULL;
    struct stat st;
    if (fstat(fd, &st) != 0) { close(fd); return NULL; }
    void *map = mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) return NULL;

    gg_cur c = {(const uint8_t *)map, (size_t)st.st_size, 0, 0};
    if (gg_u(&c, 4) != 0x46554747u) { munmap(map, (size_t)st.st_size); return NULL; }
    (void)gg_u(&c, 4); /* version */
    const uint64_t n_tensors = gg_u(&c, 8);
    const uint64_t n_kv = gg_u(&c, 8);

    gg_hparams hp;
    memset(&hp, 0, sizeof hp);
    hp.eps = 1e-6f;
    hp.theta = 10000.0f;
    hp.alignment = 32;
    for (uint64_t i = 0; i < n_kv && !c.err; ++i) {
        char key[256];
        gg_str(&c, key, sizeof key);
        const uint32_t t = (uint32_t)gg_u(&c, 4);
        if (t == 8) { gg_str(&c, NULL, 0); continue; }
        if (t == 9) {
            const uint32_t et = (uint32_t)gg_u(&c, 4);
            const uint64_t cnt = gg_u(&c, 8);
            for (uint64_t e = 0; e < cnt && !c.err; ++e) {
                if (et == 8) gg_str(&c, NULL, 0);
                else {
                    int sz = gg_scalar_size(et);
                    if (sz < 0) { c.err = 1; break; }
                    c.pos += (size_t)sz;
                }
            }
            continue;
        }
        const double v = gg_read_num(&c, t);
        /* suffix matching of architecture keys (gguf_reader.cpp:142-148, 453-491) */
        if (ends_with(key, ".block_count")) hp.n_layer = (int)v;
        else if (ends_with(key, ".context_length")) hp.n_ctx_train = (int)v;
        else if (ends_with(key, ".embedding_length")) hp.n_embd = (int)v;
        else if (ends_with(key, ".feed_forward_length")) hp.n_ff = (int)v;
        else if (ends_with(key, ".attention.head_count")) hp.n_head = (int)v;
        else if (ends_with(key, ".attention.head_count_kv")) hp.n_head_kv = (int)v;
        else if (ends_with(key, ".attention.key_length")) hp.key_length = (int)v;
        else if (ends_with(key, ".rope.freq_base")) hp.theta = (float)v;
        else if (ends_with(key, ".attention.layer_norm_rms_epsilon")) hp.eps = (float)v;
        else if (strcmp(key, "general.alignment") == 0) hp.alignment = (int)v;
    }
    gg_tensor *ts = (gg_tensor *)calloc((size_t)n_tensors, sizeof(gg_tensor));
    for (uint64_t i = 0; i < n_tensors && !c.err; ++i) {
        gg_str(&c, ts[i].name, sizeof ts[i].name);
        ts[i].n_dims = (int)gg_u(&c, 4);
        for (int d = 0; d < ts[i].n_dims && d < 4; ++d) ts[i].ne[d] = gg_u(&c, 8);
        ts[i].type = (int)gg_u(&c, 4);
        ts[i].offset = gg_u(&c, 8);
    }
    if (c.err || hp.n_layer <= 0 || hp.n_embd <= 0 || hp.n_head <= 0) {
        free(ts); munmap(map, (size_t)st.st_size); return NULL;
    }
    if (hp.n_head_kv <= 0) hp.n_head_kv = hp.n_head;
    const size_t al = (size_t)hp.alignment;
    const size_t data_off = (c.pos + al - 1) / al * al;
    const uint8_t *data0 = (const uint8_t *)map + data_off;

    mxo_model *m = (mxo_model *)calloc(1, sizeof(mxo_model));
    m->map = map;
    m->map_size = (size_t)st.st_size;
    m->hp = hp;
    m->flags = flags;
    m->form = (flags & MXO_OPEN_GGML_FORM) ? MXO_FORM_GGML : MXO_FORM_REF;
    m->nthreads = nthreads > 0 ? nthreads : 1;
    m->head_dim = hp.key_length > 0 ? hp.key_length : hp.n_embd / hp.n_head;
    m->kv_dim = m->head_dim * hp.n_head_kv;
    m->n_ctx = n_ctx;
    m->layers = (layer_w *)calloc((size_t)hp.n_layer, sizeof(layer_w));
    int bad = 0;
    bad |= bind_w(ts, n_tensors, data0, "token_embd.weight", &m->embd);
    if (bind_w(ts, n_tensors, data0, "output.weight", &m->out) != 0) m->out = m->embd;
    m->out_norm = bind_f32(ts, n_tensors, data0, "output_norm.weight");
    m->n_vocab = (int)m->out.rows;
    for (int l = 0; l < hp.n_layer; ++l) {
        char nm[96];
        layer_w *L = &m->layers[l];
#define BW(field, suffix) snprintf(nm, sizeof nm, "blk.%d." suffix, l); bad |= bind_w(ts, n_tensors, data0, nm, &L->field)
#define BF(field, suffix) snprintf(nm, sizeof nm, "blk.%d." suffix, l); L->field = bind_f32(ts, n_tensors, data0, nm)
        BW(wq, "attn_q.weight");
        BW(wk, "attn_k.weight");
        BW(wv, "attn_v.weight");
        BW(wo, "attn_output.weight");
        BW(gate, "ffn_gate.weight");
        BW(up, "ffn_up.weight");
        BW(down, "ffn_down.weight");
        BF(bq, "attn_q.bias");
        BF(bk, "attn_k.bias");
        BF(bv, "attn_v.bias");
        BF(attn_norm, "attn_norm.weight");
        BF(ffn_norm, "ffn_norm.weight");
        BF(q_norm, "attn_q_norm.weight");
        BF(k_norm, "attn_k_norm.weight");
#undef BW
#undef BF
        if (flags & MXO_OPEN_NO_QK_NORM) { L->q_norm = NULL; L->k_norm = NULL; }
    }
    free(ts);
    if (bad) { mxo_model_close(m); return NULL; }

    const size_t d = (size_t)hp.n_embd, qd = (size_t)m->head_dim * hp.n_head;
    const size_t cache_elems = (size_t)hp.n_layer * (size_t)n_ctx * (size_t)m->kv_dim;
    m->kcache = (float *)calloc(cache_elems, sizeof(float));
    m->vcache = (float *)calloc(cache_elems, sizeof(float));
    m->x = (float *)calloc(d, 4);
    m->xn = (float *)calloc(d, 4);
    m->q = (float *)calloc(qd, 4);
    m->k = (float *)calloc((size_t)m->kv_dim, 4);
    m->v = (float *)calloc((size_t)m->kv_dim, 4);
    m->att = (float *)calloc(qd, 4);
    m->o = (float *)calloc(d, 4);
    m->g = (float *)calloc((size_t)hp.n_ff, 4);
    m->u = (float *)calloc((size_t)hp.n_ff, 4);
    m->h = (float *)calloc((size_t)hp.n_ff, 4);
    m->scores = (float *)calloc((size_t)n_ctx + 1, 4);
    if (!m->kcache || !m->vcache) { mxo_model_close(m); return NULL; }
    return m;
}

void mxo_model_close(mxo_model *m)
{
    if (!m) return;
    if (m->map) munmap(m->map, m->map_size);
    free(m->layers);
    free(m->kcache); free(m->vcache);
    free(m->x); free(m->xn); free(m->q); free(m->k); free(m->v); free(m->att);
    free(m->o); free(m->g); free(m->u); free(m->h); free(m->scores);
    free(m);
}

void mxo_model_info_get(const mxo_model *m, mxo_model_info *info)
{
    memset(info, 0, sizeof *info);
    info->n_layer = m->hp.n_layer;
    info->n_embd = m->hp.n_embd;
    info->n_head = m->hp.n_head;
    info->n_head_kv = m->hp.n_head_kv;
    info->head_dim = m->head_dim;
    info->n_ff = m->hp.n_ff;
    info->n_vocab = m->n_vocab;
    info->n_ctx = m->n_ctx;
    info->eps = m->hp.eps;
    info->rope_theta = m->hp.theta;
    info->has_qk_norm = m->layers[0].q_norm != NULL;
    info->has_bias = m->layers[0].bq != NULL;
    info->tied_output = m->out.data == m->embd.data;
    info->type_wq = m->layers[0].wq.type;
    info->type_wffn_down = m->layers[0].down.type;
    info->type_output = m->out.type;
    info->type_embd = m->embd.type;
}

void mxo_model_reset(mxo_model *m) { m->pos = 0; }
int mxo_model_pos(const mxo_model *m) { return m->pos; }
int mxo_model_set_pos(mxo_model *m, int pos)
{
    if (pos < 0 || pos >= m->n_ctx) return -1;
    m->pos = pos;
    return 0;
}

static void proj(const mxo_model *m, const wt *w, const float *x, float *y)
{
    mxo_matmul_rhs_t(w->type, x, 1, w->cols, w->data, w->rows, y, m->form, m->nthreads);
}

/* One decoder layer for one token at position pos (transformer.cpp:330-755
 * with seq = 1), plus Qwen3 QK-norm after the projections and before RoPE
 * when the layer carries attn_{q,k}_norm (absent from the reference). */
static void layer_forward(mxo_model *m, int l, int pos)
{
    const layer_w *L = &m->layers[l];
    const int d = m->hp.n_embd, hd = m->head_dim, nh = m->hp.n_head, nkv = m->hp.n_head_kv;
    const int kvd = m->kv_dim;
    const float eps = m->hp.eps;
    const int neox = (m->flags & MXO_OPEN_ROPE_NEOX) != 0;

    mxo_rmsnorm(m->x, L->attn_norm, m->xn, (size_t)d, eps);
    proj(m, &L->wq, m->xn, m->q);
    proj(m, &L->wk, m->xn, m->k);
    proj(m, &L->wv, m->xn, m->v);
    if (L->bq) for (int i = 0; i < nh * hd; ++i) m->q[i] += L->bq[i];
    if (L->bk) for (int i = 0; i < kvd; ++i) m->k[i] += L->bk[i];
    if (L->bv) for (int i = 0; i < kvd; ++i) m->v[i] += L->bv[i];
    if (L->q_norm) for (int h = 0; h < nh; ++h) mxo_rmsnorm(m->q + h * hd, L->q_norm, m->q + h * hd, (size_t)hd, eps);
    if (L->k_norm) for (int h = 0; h < nkv; ++h) mxo_rmsnorm(m->k + h * hd, L->k_norm, m->k + h * hd, (size_t)hd, eps);
    /* the cache is a ring of n_ctx rows (kv_cache.cpp:50-75): `cached` rows
     * are held (cache->lengths, which stops growing at n_ctx), the oldest at
     * row `head` once the ring is full; RoPE takes start_pos = cached
     * (transformer.cpp:506), so positions past n_ctx all rotate by n_ctx */
    const int cached = pos < m->n_ctx ? pos : m->n_ctx;
    const int head = pos < m->n_ctx ? 0 : (pos - m->n_ctx) % m->n_ctx;
    mxo_rope(m->q, (size_t)nh, (size_t)hd, 0, (size_t)cached, m->hp.theta, neox);
    mxo_rope(m->k, (size_t)nkv, (size_t)hd, 0, (size_t)cached, m->hp.theta, neox);

    float *kc = m->kcache + (size_t)l * m->n_ctx * kvd;
    float *vc = m->vcache + (size_t)l * m->n_ctx * kvd;
    if (m->flags & MXO_OPEN_KV_FP16) {
        /* the GPU cache stores fp16; the current token is read back from it */
        for (int i = 0; i < kvd; ++i) {
            m->k[i] = mxo_fp16_to_fp32(mxo_fp32_to_fp16(m->k[i]));
            m->v[i] = mxo_fp16_to_fp32(mxo_fp32_to_fp16(m->v[i]));
        }
    }

    /* attention (transformer.cpp:529-629): scores over the cached rows,
     * oldest first (row (head + j) % n_ctx, backend_vec_dot_rows_ring), plus
     * the current row, double-accumulated dots, x 1/sqrt(hd) in float,
     * softmax, then V: cached rows accumulate out += w*v in float, the
     * current row is a double dot (cpu_vec_mul_rows_cols) added last. */
    const int group = nh / nkv;
    const float scale = 1.0f / sqrtf((float)hd);
    const int J = cached + 1;
    for (int h = 0; h < nh; ++h) {
        int kvh = h / (group > 0 ? group : 1);
        if (kvh > nkv - 1) kvh = nkv - 1;
        const float *qh = m->q + h * hd;
        for (int j = 0; j < J; ++j) {
            const float *kr = j < cached ? kc + (size_t)((head + j) % m->n_ctx) * kvd + kvh * hd : m->k + kvh * hd;
            double acc = 0.0;
            for (int t = 0; t < hd; ++t) acc += (double)qh[t] * (double)kr[t];
            m->scores[j] = (float)acc;
        }
        for (int j = 0; j < J; ++j) m->scores[j] *= scale;
        mxo_softmax(m->scores, (size_t)J);
        float *out = m->att + h * hd;
        for (int t = 0; t < hd; ++t) out[t] = 0.0f;
        for (int j = 0; j < cached; ++j) {
            const float w = m->scores[j];
            const float *vr = vc + (size_t)((head + j) % m->n_ctx) * kvd + kvh * hd;
            for (int t = 0; t < hd; ++t) out[t] = fmaf(w, vr[t], out[t]);
        }
        const float wc = m->scores[cached];
        for (int t = 0; t < hd; ++t) out[t] += (float)((double)wc * (double)m->v[kvh * hd + t]);
    }
    /* kvcache_append: the next free row, or the oldest one once full */
    const int row = pos < m->n_ctx ? pos : head;
    memcpy(kc + (size_t)row * kvd, m->k, sizeof(float) * (size_t)kvd);
    memcpy(vc + (size_t)row * kvd, m->v, sizeof(float) * (size_t)kvd);

    proj(m, &L->wo, m->att, m->o);
    for (int i = 0; i < d; ++i) m->x[i] += m->o[i];

    mxo_rmsnorm(m->x, L->ffn_norm, m->xn, (size_t)d, eps);
    proj(m, &L->gate, m->xn, m->g);
    proj(m, &L->up, m->xn, m->u);
    for (int i = 0; i < m->hp.n_ff; ++i) m->h[i] = mxo_silu(m->g[i]) * m->u[i];
    proj(m, &L->down, m->h, m->o);
    for (int i = 0; i < d; ++i) m->x[i] += m->o[i];
}

int mxo_model_step(mxo_model *m, int token, float *logits, float *hidden_trace)
{
    if (!m || token < 0 || (size_t)token >= m->embd.rows || m->pos == INT_MAX) return -1;
    const int d = m->hp.n_embd;
    /* token_embedding_row_into: dequantize row `token` (minxfmr.cpp:210-343) */
    if (m->embd.type == MXO_F32)
        memcpy(m->x, m->embd.data + (size_t)token * d * 4, sizeof(float) * (size_t)d);
    else
        mxo_dequant_rows(m->embd.type, m->embd.data + (size_t)token * mxo_row_bytes(m->embd.type, (size_t)d), 1,
                         (size_t)d, m->x, m->form);
    for (int l = 0; l < m->hp.n_layer; ++l) {
        layer_forward(m, l, m->pos);
        if (hidden_trace) memcpy(hidden_trace + (size_t)l * d, m->x, sizeof(float) * (size_t)d);
    }
    m->pos++;
    /* apply_final_norm_inplace (minxfmr.cpp:522-531) then the lm-head */
    mxo_rmsnorm(m->x, m->out_norm, m->xn, (size_t)d, m->hp.eps);
    if (hidden_trace) memcpy(hidden_trace + (size_t)m->hp.n_layer * d, m->xn, sizeof(float) * (size_t)d);
    if (logits) proj(m, &m->out, m->xn, logits);
    return 0;
}
