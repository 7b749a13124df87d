"""Parity of the HIP dequant / GEMV kernels with the CPU oracle (GPU).

Bars: dequantized weights bit-exact; GEMV fp32 output within 1e-3 relative
of the CPU kernel, tested per element as |y - y_ref| <= 1e-3 * |y_ref| +
2^-20 * max|y_ref|, plus a global max-error / max-value bound of 2^-20.
The floor keeps outputs that cancel to ~0 from demanding unbounded relative
accuracy; at 2^-20 (about 1e-6) of the largest output it is an fp32-level
bound: summation-order differences of fp32 dot products at these sizes are
about 1e-8 of it, while staging x with 16 bits (half a unit of 2^-16 of
each 32-element sub-block's largest |x|) misses it by an order of magnitude.
The quantized kernels stage x as 24-bit block fixed point and use the
weights exactly.  For F32 rows and the F16 / Q6_K rows the reference turns
into F32 at load, the reference sums each row in fp32 and is itself only
accurate to about 1e-6 of max|y| at K = 4096: there the per-element check
adds the worst-case bound of that sum, and the 2^-20 bound is taken against
the float64 product (check_vs_oracle).
"""
from __future__ import annotations

import numpy as np
import pytest

import mxo

pytestmark = pytest.mark.gpu

TYPES = {"Q4_K": mxo.Q4_K, "Q5_K": mxo.Q5_K, "Q6_K": mxo.Q6_K, "Q8_0": mxo.Q8_0, "Q5_0": mxo.Q5_0, "F16": mxo.F16,
         "F32": mxo.F32}


def same_bits(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))))


def random_blocks(rng, t, nblocks):
    be, bb = mxo.BLOCK[t]
    raw = rng.integers(0, 256, size=(nblocks, bb), dtype=np.uint8)
    if t in (mxo.Q4_K, mxo.Q5_K):
        raw[:, 0:4] = (rng.standard_normal((nblocks, 2)) * 0.01).astype(np.float16).view(np.uint8)
    elif t in (mxo.Q8_0, mxo.Q5_0):
        raw[:, 0:2] = (rng.standard_normal((nblocks, 1)) * 0.01).astype(np.float16).view(np.uint8)
    elif t == mxo.Q6_K:
        raw[:, 208:210] = (rng.standard_normal((nblocks, 1)) * 0.01).astype(np.float16).view(np.uint8)
    return raw.reshape(-1)


@pytest.mark.parametrize("name", ["Q4_K", "Q5_K", "Q6_K", "Q8_0", "Q5_0"])
@pytest.mark.parametrize("form", [mxo.FORM_REF, mxo.FORM_GGML])
def test_dequant_bit_exact_random_blocks(mxh, name, form):
    t = TYPES[name]
    rng = np.random.default_rng(100 + t + 7 * form)
    rows, cols = 37, 256 * 6
    raw = random_blocks(rng, t, rows * cols // mxo.BLOCK[t][0])
    buf = mxh.DeviceBuffer.from_array(raw)
    got = mxh.dequant(t, buf, rows, cols, form)
    want = mxo.dequant(t, raw, rows, cols, form)
    assert same_bits(got, want)


def test_dequant_bit_exact_any_bits_including_nan_inf(mxh):
    """Unconstrained bytes: fp16 d/dmin may be subnormal, inf or NaN."""
    rng = np.random.default_rng(5)
    for t in (mxo.Q4_K, mxo.Q5_K, mxo.Q6_K, mxo.Q8_0, mxo.Q5_0):
        be, bb = mxo.BLOCK[t]
        raw = rng.integers(0, 256, size=(64 * bb,), dtype=np.uint8)
        buf = mxh.DeviceBuffer.from_array(raw)
        for form in (0, 1):
            assert same_bits(mxh.dequant(t, buf, 1, 64 * be, form), mxo.dequant(t, raw, 1, 64 * be, form))


def test_f16_decode_exhaustive(mxh):
    h = np.arange(65536, dtype=np.uint16)
    buf = mxh.DeviceBuffer.from_array(h.view(np.uint8))
    got = mxh.dequant(mxo.F16, buf, 1, 65536)
    want = mxo.dequant(mxo.F16, h.view(np.uint8), 1, 65536)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))  # NaN payloads too


FLOOR = 2.0 ** -20


def check_close(got, want, rtol=1e-3, exact=None, ref_slack=None):
    """Per element against the CPU kernel `want` within rtol (plus the floor,
    plus `ref_slack`, a bound on the CPU kernel's own rounding where it sums
    a whole row in fp32), and globally within FLOOR of `exact` (the float64
    product; the CPU kernel itself where its accumulation is exact enough)."""
    scale = float(np.abs(want).max()) or 1.0
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    slack = 0.0 if ref_slack is None else ref_slack
    assert np.all(err <= rtol * np.abs(want) + FLOOR * scale + slack), f"max err {err.max()} scale {scale}"
    ex = want.astype(np.float64) if exact is None else exact
    gerr = float(np.abs(got.astype(np.float64) - ex).max()) / (float(np.abs(ex).max()) or 1.0)
    assert gerr <= FLOOR, f"max err / max value = {gerr}"


# F32 rows, and the F16 / Q6_K rows the reference converts to F32 at load,
# are summed over the whole row in fp32 by the reference
# (backend_runtime.cpp:413-425, an OpenMP SIMD float reduction; the oracle
# sums in order): its own rounding, up to K 2^-24 sum|x w| per output, is
# about 1e-6 of max|y| at K = 4096, so the fp32-level bound is taken against
# the float64 product of the same weights instead.
FP32_ROW_SUM = (mxo.F32, mxo.F16, mxo.Q6_K)


def check_vs_oracle(got, want, t, w, x, n, k, form=mxo.FORM_REF):
    if t not in FP32_ROW_SUM:
        return check_close(got, want)
    wd = mxo.dequant(t, w, n, k, form).astype(np.float64)
    exact = wd @ x.astype(np.float64)
    slack = k * 2.0 ** -24 * (np.abs(wd) @ np.abs(x.astype(np.float64)))
    check_close(got, want, exact=exact, ref_slack=slack)


def run_gemv(mxh, t, w, x, n, k, form=mxo.FORM_REF):
    wb = mxh.DeviceBuffer.from_array(w)
    xb = mxh.DeviceBuffer.from_array(x)
    yb = mxh.DeviceBuffer(n * 4)
    mxh.gemv(t, wb, xb, yb, n, k, form)
    return yb.download(np.float32, n)


GEMV_CASES = [
    ("Q4_K", 4096, 4096), ("Q4_K", 12288, 4096), ("Q4_K", 4096, 12288), ("Q4_K", 151936, 4096),
    ("Q4_K", 1, 256), ("Q4_K", 7, 512), ("Q4_K", 1000, 14336), ("Q4_K", 24, 2816),
    ("Q5_K", 1024, 4096), ("Q5_K", 4096, 14336), ("Q5_K", 9, 256),
    ("Q8_0", 151936, 4096), ("Q8_0", 1024, 1024), ("Q8_0", 3, 32), ("Q8_0", 5, 96), ("Q8_0", 1, 3072),
    ("Q5_0", 256, 512), ("Q5_0", 7, 96), ("F32", 100, 512), ("F32", 3, 32),
    # Q6_K in the GGUF block order (2-aligned 210-byte blocks: odd rows and
    # odd blocks start at 2 mod 4), the llama.cpp Q4_K_M head and down shapes
    ("Q6_K", 151936, 4096), ("Q6_K", 4096, 14336), ("Q6_K", 7, 256), ("Q6_K", 33, 1280),
    ("F16", 300, 4096), ("F16", 3, 32), ("F16", 1000, 14336),
]


@pytest.mark.parametrize("name,n,k", GEMV_CASES, ids=[f"{a}-{b}x{c}" for a, b, c in GEMV_CASES])
def test_gemv_vs_oracle(mxh, name, n, k):
    t = TYPES[name]
    rng = np.random.default_rng(n * 31 + k)
    wf = rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)
    w = mxo.quantize(t, wf)
    x = rng.standard_normal(k, dtype=np.float32)
    for form in ((mxo.FORM_REF, mxo.FORM_GGML) if t in (mxo.Q4_K, mxo.Q5_K) and n * k <= 1 << 24 else (mxo.FORM_REF,)):
        got = run_gemv(mxh, t, w, x, n, k, form)
        want = mxo.matmul_rhs_t(t, x, w, n, form)[0]
        check_vs_oracle(got, want, t, w, x, n, k, form)


@pytest.mark.parametrize("name", ["Q4_K", "Q5_K", "Q6_K", "Q8_0", "Q5_0", "F16", "F32"])
def test_gemv_non_finite_x_propagates(mxh, name):
    """A NaN in x gives NaN outputs and an infinity non-finite ones, as the
    reference's fp32 products do (x * w summed over every block of a row)."""
    t = TYPES[name]
    rng = np.random.default_rng(9)
    n, k = 70, 512
    w = mxo.quantize(t, rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    for bad in (np.nan, np.inf):
        x = rng.standard_normal(k, dtype=np.float32)
        x[300] = bad
        got = run_gemv(mxh, t, w, x, n, k)
        want = mxo.matmul_rhs_t(t, x, w, n)[0]
        assert not np.isfinite(want).any()
        if bad != bad:
            assert np.isnan(got).all(), got[:8]
        else:
            assert not np.isfinite(got).any(), got[:8]


TILE_CASES = [("Q4_K", 12288, 4096, True), ("Q4_K", 1000, 14336, True), ("Q4_K", 24, 2816, True),
              ("Q5_K", 4096, 14336, True), ("Q8_0", 1024, 4096, True),
              ("Q6_K", 151936, 4096, True), ("Q6_K", 1000, 14336, True), ("Q6_K", 3, 2048, True),
              ("Q6_K", 12, 1024, False), ("Q8_0", 3, 32, False), ("Q5_0", 7, 256, False), ("F16", 8, 512, False)]


@pytest.mark.parametrize("name,n,k,tiles", TILE_CASES, ids=[f"{a}-{b}x{c}" for a, b, c, _ in TILE_CASES])
def test_tiled_rows_give_identical_gemv(mxh, name, n, k, tiles):
    """mxh_tile_rows regroups rows in place into the tiled order (Q4_K, Q5_K,
    Q8_0 with k a multiple of 256 up to 15360; Q6_K with k a multiple of 2048,
    which keeps its 210-byte-block rows 16-byte aligned) and returns the id
    mxh_gemv then takes; the products are bit-identical to those over the
    GGUF rows.  Other shapes and types (Q8_0 rows of 32, Q6_K rows of 1024,
    Q5_0, F16) are left as they are and keep their id; every Q4_K shape the
    GEMV takes is tileable."""
    t = TYPES[name]
    rng = np.random.default_rng(n * 7 + k)
    w = mxo.quantize(t, rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    x = rng.standard_normal(k, dtype=np.float32)
    wb, xb, yb = mxh.DeviceBuffer.from_array(w), mxh.DeviceBuffer.from_array(x), mxh.DeviceBuffer(4 * n)
    mxh.gemv(t, wb, xb, yb, n, k)
    y0 = yb.download(np.float32, n)
    tt = mxh.tile_rows(t, wb, n, k)
    assert tt == ((t | mxh.TILED_FLAG) if tiles else t)
    if tiles:
        assert not np.array_equal(wb.download(np.uint8, w.size), w.ravel()), "rows were not regrouped"
    mxh.gemv(tt, wb, xb, yb, n, k)
    assert np.array_equal(yb.download(np.float32, n), y0)
    if not tiles:
        with pytest.raises(mxh.MxhError, match="tiled form"):
            mxh.gemv(t | mxh.TILED_FLAG, wb, xb, yb, n, k)
    for b in (wb, xb, yb):
        b.close()


def test_gemv_reference_kat_blocks(mxh):
    """Crafted blocks of the reference parity test, every row the same, x = ones."""
    import json
    from pathlib import Path
    kat = json.loads((Path(__file__).parent / "golden" / "reference_kat.json").read_text())
    for name in ("Q4_K", "Q5_0", "Q8_0"):
        t = TYPES[name]
        be = mxo.BLOCK[t][0]
        blk = np.frombuffer(bytes.fromhex(kat[name]["block_hex"]), np.uint8)
        y = run_gemv(mxh, t, np.tile(blk, be), np.ones(be, np.float32), be, be)
        assert np.all(y == kat[name]["ones_dot"]), (name, y[:4])


def test_matmul_rhs_t_multi_row(mxh):
    rng = np.random.default_rng(77)
    m, n, k = 5, 300, 1024
    w = mxo.quantize(mxo.Q4_K, rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    a = rng.standard_normal((m, k), dtype=np.float32)
    got = mxh.host_matmul_rhs_t(mxo.Q4_K, a, w, n)
    want = mxo.matmul_rhs_t(mxo.Q4_K, a, w, n)
    check_close(got, want)


def test_host_vector_ops(mxh):
    import ctypes as C
    lib = mxh.lib
    rng = np.random.default_rng(3)
    K, N, stride = 128, 50, 160
    vec = rng.standard_normal(K).astype(np.float32)
    rows = rng.standard_normal(N * stride).astype(np.float32)
    out = np.empty(N, np.float32)
    mxh.check(lib.mxh_host_vec_dot_rows(mxh.ptr(vec), mxh.ptr(rows), mxh.ptr(out), K, N, stride))
    want = rows.reshape(N, stride)[:, :K].astype(np.float64) @ vec.astype(np.float64)
    np.testing.assert_allclose(out, want.astype(np.float32), rtol=1e-6, atol=1e-6)
    # ring: head 13 of seq_max N, len 40
    head, ln = 13, 40
    out2 = np.empty(ln, np.float32)
    mxh.check(lib.mxh_host_vec_dot_rows_ring(mxh.ptr(vec), mxh.ptr(rows), head, N, ln, K, stride, mxh.ptr(out2)))
    np.testing.assert_allclose(out2, want[[(head + j) % N for j in range(ln)]].astype(np.float32), rtol=1e-6, atol=1e-6)
    # rows x cols
    v2 = rng.standard_normal(N).astype(np.float32)
    out3 = np.empty(K, np.float32)
    mxh.check(lib.mxh_host_vec_mul_rows_cols(mxh.ptr(v2), mxh.ptr(rows), mxh.ptr(out3), N, K, stride))
    want3 = v2.astype(np.float64) @ rows.reshape(N, stride)[:, :K].astype(np.float64)
    np.testing.assert_allclose(out3, want3.astype(np.float32), rtol=1e-6, atol=1e-6)
    out4 = np.empty(K, np.float32)
    mxh.check(lib.mxh_host_matvec_strided(mxh.ptr(v2), mxh.ptr(rows), mxh.ptr(out4), N, K, stride))
    np.testing.assert_array_equal(out4, out3)
    # F32 matmul known answer (tests/test_cuda_quantized_matmul.cpp:57-90)
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    c = np.empty((2, 2), np.float32)
    mxh.check(lib.mxh_host_matmul_f32(mxh.ptr(a), mxh.ptr(b), mxh.ptr(c), 2, 3, 2))
    assert c.tolist() == [[58, 64], [139, 154]]


def test_argument_errors_are_reported_not_launched(mxh):
    buf = mxh.DeviceBuffer(1 << 16)
    xb = mxh.DeviceBuffer(4096)
    yb = mxh.DeviceBuffer(4096)
    lib = mxh.lib
    assert lib.mxh_gemv(mxo.Q4_K, buf.ptr, xb.ptr, yb.ptr, 4, 100, 0) == -1      # k not a block multiple
    assert b"blocks" in lib.mxh_last_error()
    assert lib.mxh_gemv(mxo.Q4_K, buf.ptr + 4, xb.ptr, yb.ptr, 4, 256, 0) == -1  # misaligned weights
    assert lib.mxh_gemv(99, buf.ptr, xb.ptr, yb.ptr, 4, 256, 0) == -1            # unknown type
    assert lib.mxh_gemv(mxo.Q4_K, buf.ptr, xb.ptr, yb.ptr, 0, 256, 0) == -1      # empty
    assert lib.mxh_dequant(mxo.Q4_K, buf.ptr, yb.ptr, 1, 100, 0) == -1
