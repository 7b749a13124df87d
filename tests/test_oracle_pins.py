"""Pins of the CPU oracle (oracle/mxo.c) — CPU only.

Each oracle function is checked against something it does not itself
compute: the reference's known-answer tests, vectors produced by the
reference's own CPU code (tests/golden/, and oracle/_ref when it is built
here), IEEE conversions from numpy, closed forms, and brute force in float64.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

import mxo

GOLD = Path(__file__).resolve().parent / "golden"
KAT = json.loads((GOLD / "reference_kat.json").read_text())
VEC = np.load(GOLD / "ref_vectors.npz")
REF = mxo.load_ref()


def same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | nan))


# ---- known-answer tests held by the reference -----------------------------

def test_q4k_kat_reference_form():
    """tests/test_cuda_quantized_matmul.cpp:18-42: out[128] == -1 (CPU form)."""
    blk = np.frombuffer(bytes.fromhex(KAT["Q4_K"]["block_hex"]), np.uint8)
    y = mxo.dequant(mxo.Q4_K, blk, 1, 256, mxo.FORM_REF)[0]
    assert y[128] == -1.0
    assert np.array_equal(y, np.array(KAT["Q4_K"]["dequant"], np.float32))
    # closed form: sub-block 4 has sc = 16, m = 17 -> 16*q - 17; all else 0
    want = np.zeros(256, np.float32)
    want[128:160] = -17.0
    want[128] = -1.0
    assert np.array_equal(y, want)


def test_q4k_kat_ggml_form():
    """The ggml decoder gives -17 at [128] where the reference CPU form gives
    -1 (test_cuda_quantized_matmul.cpp:18-42 pins -1): sc = 0, m = 17."""
    blk = np.frombuffer(bytes.fromhex(KAT["Q4_K"]["block_hex"]), np.uint8)
    y = mxo.dequant(mxo.Q4_K, blk, 1, 256, mxo.FORM_GGML)[0]
    want = np.zeros(256, np.float32)
    want[128:160] = -17.0
    assert np.array_equal(y, want)


@pytest.mark.parametrize("name,t,be", [("Q4_K", mxo.Q4_K, 256), ("Q5_0", mxo.Q5_0, 32), ("Q8_0", mxo.Q8_0, 32)])
def test_parity_kat_ones_dot(name, t, be):
    """tests/test_cuda_quant_kernel_parity.cpp:26-67: crafted block in every row, A = ones."""
    blk = np.frombuffer(bytes.fromhex(KAT[name]["block_hex"]), np.uint8)
    y = mxo.matmul_rhs_t(t, np.ones(be, np.float32), np.tile(blk, be), be)[0]
    assert np.all(y == KAT[name]["ones_dot"])
    closed = {"Q4_K": -1 + 31 * -17, "Q5_0": -1 + 31 * -16, "Q8_0": -1}[name]
    assert KAT[name]["ones_dot"] == closed


def test_f32_matmul_kat():
    """tests/test_cuda_quantized_matmul.cpp:57-90 expects [[58,64],[139,154]]."""
    a = np.array(KAT["F32_matmul"]["a"], np.float32)
    b = np.array(KAT["F32_matmul"]["b"], np.float32)
    out = mxo.matmul_rhs_t(mxo.F32, a, np.ascontiguousarray(b.T).view(np.uint8), 2)
    assert np.array_equal(out, np.array(KAT["F32_matmul"]["c"], np.float32))


# ---- fp16 -------------------------------------------------------------------

def test_fp16_exhaustive_vs_ieee():
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    # through the F16 row decoder so no float->double conversion touches NaN bits
    got = mxo.dequant(mxo.F16, h.view(np.uint8), 1, 65536)[0]
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # NaN payloads: the reference keeps frac << 13 with the quiet bit as given
    frac = (h[nan] & 0x3FF).astype(np.uint32)
    sign = (h[nan].astype(np.uint32) >> 15) << 31
    assert np.array_equal(got[nan].view(np.uint32), sign | 0x7F800000 | (frac << 13))


@pytest.mark.skipif(REF is None, reason="reference build (oracle/_ref) not present")
def test_fp16_exhaustive_vs_reference():
    for v in range(65536):
        a, b = mxo.fp16_to_fp32(v), REF.ref_fp16_to_fp32(v)
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32) or (np.isnan(a) and np.isnan(b))


def test_fp32_to_fp16_rne_vs_numpy():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10 ** rng.uniform(-9, 5, 20000),
                        np.array([0.0, -0.0, 65504, 65519.99, 65520, 1e-8, 5.96e-8, 2.98e-8, 2.99e-8, np.inf,
                                  -np.inf], np.float32)]).astype(np.float32)
    want = x.astype(np.float16).view(np.uint16)
    got = np.array([mxo.lib.mxo_fp32_to_fp16(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, want)


# ---- block dequant -----------------------------------------------------------

@pytest.mark.parametrize("t,be", [(mxo.Q4_K, 256), (mxo.Q8_0, 32), (mxo.Q5_0, 32)])
def test_dequant_random_blocks_vs_reference_vectors(t, be):
    blocks = VEC[f"blocks_{t}"]
    got = mxo.dequant(t, blocks.reshape(-1), 1, be * len(blocks), mxo.FORM_REF).reshape(len(blocks), be)
    assert same_bits(got, VEC[f"dequant_{t}"])


def _q4k_closed_form(blk: np.ndarray, ggml: bool) -> np.ndarray:
    d = float(blk[0:2].view(np.float16)[0])
    dm = float(blk[2:4].view(np.float16)[0])
    s = blk[4:16].astype(np.int64)
    out = np.empty(256)
    for j in range(8):
        if j < 4:
            sc, m = s[j] & 63, s[j + 4] & 63
        else:
            sc = (s[j + 4] & 15) | ((s[j - 4 if ggml else j] >> 6) << 4)
            m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4)
        g, hi = divmod(j, 2)
        q = blk[16 + 32 * g: 48 + 32 * g].astype(np.int64)
        q = (q >> 4) if hi else (q & 15)
        out[32 * j: 32 * j + 32] = (d * sc) * q - dm * m  # float64: exact products, one rounding below
    return out.astype(np.float32)


@pytest.mark.parametrize("ggml", [False, True])
def test_q4k_dequant_closed_form(ggml):
    """value = (d*sc)*q - dmin*m: every product is exact, so float64 then one
    rounding to float32 must equal the oracle bit for bit."""
    rng = np.random.default_rng(7)
    for _ in range(200):
        blk = rng.integers(0, 256, 144, dtype=np.uint8)
        blk[0:4] = (rng.standard_normal(2) * 0.05).astype(np.float16).view(np.uint8)
        got = mxo.dequant(mxo.Q4_K, blk, 1, 256, mxo.FORM_GGML if ggml else mxo.FORM_REF)[0]
        assert same_bits(got, _q4k_closed_form(blk, ggml))


def test_q5k_reduces_to_q4k_without_high_bits():
    """Q5_K with qh == 0 decodes exactly like the Q4_K block with the same d,
    dmin, scales and nibbles; setting bit j of qh[i] adds exactly 16*d*sc_j to
    element 32j+i (the published ggml layout)."""
    rng = np.random.default_rng(11)
    for form in (mxo.FORM_REF, mxo.FORM_GGML):
        for _ in range(100):
            q4 = rng.integers(0, 256, 144, dtype=np.uint8)
            q4[0:4] = (rng.standard_normal(2) * 0.05).astype(np.float16).view(np.uint8)
            q5 = np.zeros(176, np.uint8)
            q5[0:16] = q4[0:16]
            q5[48:176] = q4[16:144]
            y4 = mxo.dequant(mxo.Q4_K, q4, 1, 256, form)[0]
            y5 = mxo.dequant(mxo.Q5_K, q5, 1, 256, form)[0]
            assert same_bits(y4, y5)
            i, j = int(rng.integers(0, 32)), int(rng.integers(0, 8))
            q5b = q5.copy()
            q5b[16 + i] |= 1 << j
            y5b = mxo.dequant(mxo.Q5_K, q5b, 1, 256, form)[0]
            diff = np.nonzero(~((y5b == y5) | (np.isnan(y5b) & np.isnan(y5))))[0]
            e = 32 * j + i
            assert set(diff.tolist()) <= {e}
            assert same_bits(y5b[e:e + 1], np.array([_q5k_elem(q5b, e, form)], np.float32))


def _q5k_elem(blk, e, form):
    j, i = divmod(e, 32)
    d = float(blk[0:2].view(np.float16)[0])
    dm = float(blk[2:4].view(np.float16)[0])
    s = blk[4:16].astype(np.int64)
    if j < 4:
        sc, m = s[j] & 63, s[j + 4] & 63
    else:
        sc = (s[j + 4] & 15) | ((s[j - 4 if form == mxo.FORM_GGML else j] >> 6) << 4)
        m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4)
    g, hi = divmod(j, 2)
    qb = int(blk[48 + 32 * g + i])
    q = (qb >> 4) if hi else (qb & 15)
    q |= ((int(blk[16 + i]) >> j) & 1) << 4
    return np.float32((d * sc) * q - dm * m)


def _q6k_closed_form(blk: np.ndarray) -> np.ndarray:
    """The published Q6_K layout in numpy: element 128h + 32g + l (l < 32)
    has the code nibble of ql[64h + 32(g & 1) + l] (low for g < 2) with the
    2-bit field g of qh[32h + l] above it, minus 32, scaled by
    d * scales[e // 16]; the products are exact in float64, so one rounding
    to float32 gives the value (d * sc) * q the reference computes in float."""
    ql, qh = blk[0:128].astype(np.int64), blk[128:192].astype(np.int64)
    sc = blk[192:208].view(np.int8).astype(np.float64)
    d = float(blk[208:210].view(np.float16)[0])
    out = np.empty(256)
    for e in range(256):
        h, r = divmod(e, 128)
        g, l = divmod(r, 32)
        nib = ql[64 * h + 32 * (g & 1) + l]
        nib = (nib >> 4) if g >= 2 else (nib & 15)
        q = nib | (((qh[32 * h + l] >> (2 * g)) & 3) << 4)
        out[e] = (d * sc[e // 16]) * (q - 32)
    with np.errstate(invalid="ignore", over="ignore"):
        return out.astype(np.float32)


def test_q6k_dequant_closed_form():
    rng = np.random.default_rng(61)
    for _ in range(100):
        blk = rng.integers(0, 256, 210, dtype=np.uint8)
        blk[208:210] = (rng.standard_normal(1) * 0.05).astype(np.float16).view(np.uint8)
        assert same_bits(mxo.dequant(mxo.Q6_K, blk, 1, 256)[0], _q6k_closed_form(blk))


@pytest.mark.skipif(REF is None, reason="oracle/_ref not built (reference tree absent)")
def test_q6k_and_f16_decode_vs_reference_loader():
    """The reference converts Q6_K and F16 tensors to F32 when it loads them
    (gguf_reader.cpp:905-1008, :759-785); its own functions, compiled under
    oracle/_ref, give the same bits as the oracle for blocks with any bytes
    (fp16 d subnormal, inf or NaN), for quantized rows, and for every fp16
    value."""
    rng = np.random.default_rng(62)
    rows, cols = 6, 1024
    for raw in (rng.integers(0, 256, rows * cols // 256 * 210, dtype=np.uint8),
                mxo.quantize(mxo.Q6_K, rng.standard_normal((rows, cols)).astype(np.float32) * 0.02)):
        want = np.empty((rows, cols), np.float32)
        assert REF.ref_gguf_to_f32(14, raw.ctypes.data, raw.size, rows, cols, want.ctypes.data) == 0
        assert same_bits(mxo.dequant(mxo.Q6_K, raw, rows, cols), want)
    h = np.arange(65536, dtype=np.uint16)
    want = np.empty(65536, np.float32)
    assert REF.ref_gguf_to_f32(1, h.ctypes.data, h.nbytes, 1, 65536, want.ctypes.data) == 0
    got = mxo.dequant(mxo.F16, h.view(np.uint8), 1, 65536)[0]
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_type41_is_the_byte_value():
    """GGUF type 41 holds one byte per element (the reference's size rule,
    gguf_reader.cpp:575-584, gives it rows * cols bytes) and its reader
    takes each byte as the weight, 0..255 (:1023-1041); the oracle's decode
    is that closed form for every byte value, and its matmul over such rows
    equals the matmul over the widened F32 rows."""
    b = np.arange(256, dtype=np.uint8)
    assert np.array_equal(mxo.dequant(mxo.Q1_0, b, 1, 256)[0], np.arange(256, dtype=np.float32))
    rng = np.random.default_rng(41)
    raw = rng.integers(0, 256, 7 * 96, dtype=np.uint8)
    a = rng.standard_normal((3, 96)).astype(np.float32)
    wide = raw.astype(np.float32).reshape(7, 96)
    assert same_bits(mxo.matmul_rhs_t(mxo.Q1_0, a, raw, 7), mxo.matmul_rhs_t(mxo.F32, a, wide, 7))
    # and the F32 rows' float fma chain is the product to fp32 rounding
    assert np.allclose(mxo.matmul_rhs_t(mxo.Q1_0, a, raw, 7), a.astype(np.float64) @ wide.T.astype(np.float64),
                       rtol=1e-6, atol=1e-4)


@pytest.mark.skipif(REF is None, reason="oracle/_ref not built (reference tree absent)")
def test_type41_decode_vs_reference_loader():
    """The reference's own type-41 reader (gguf_reader.cpp:1010-1098),
    compiled under oracle/_ref, gives the same bits as the oracle for every
    byte value, on rows of several lengths."""
    rng = np.random.default_rng(4141)
    for rows, cols in ((1, 256), (5, 300), (16, 4096)):
        raw = rng.integers(0, 256, rows * cols, dtype=np.uint8)
        want = np.empty((rows, cols), np.float32)
        assert REF.ref_gguf_to_f32(41, raw.ctypes.data, raw.size, rows, cols, want.ctypes.data) == 0
        assert same_bits(mxo.dequant(mxo.Q1_0, raw, rows, cols), want)


@pytest.mark.parametrize("t,tol", [(mxo.Q8_0, 0.008), (mxo.Q4_K, 0.12), (mxo.Q5_K, 0.06), (mxo.Q5_0, 0.06),
                                   (mxo.Q6_K, 0.03)])
def test_quantizer_round_trip(t, tol):
    """Generators used for synthetic models: relative RMS error of the round
    trip, decoded with the ggml scale form the quantizer packs for (the
    reference CPU form misreads sub-blocks 4..7 of standard GGUF K-quants)."""
    rng = np.random.default_rng(3)
    w = rng.standard_normal((8, 1024)).astype(np.float32) * 0.02
    q = mxo.quantize(t, w)
    assert q.nbytes == mxo.row_bytes(t, 1024) * 8
    back = mxo.dequant(t, q, 8, 1024, mxo.FORM_GGML)
    err = np.sqrt(np.mean((back - w) ** 2)) / np.sqrt(np.mean(w ** 2))
    assert err < tol, err


# ---- rhs-transposed matmul ----------------------------------------------------

@pytest.mark.parametrize("key", [k[:-4] for k in VEC.files if k.startswith("mm_") and k.endswith("_out")])
def test_matmul_vs_reference_vectors(key):
    t, k, n, m = (int(v) for v in key.split("_")[1:5])
    got = mxo.matmul_rhs_t(t, VEC[key + "_a"], VEC[key + "_w"], n)
    want = VEC[key + "_out"]
    if t == mxo.Q4_K:
        # double accumulation of exact products in block order: bit-exact
        assert same_bits(got, want)
    else:
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("t", [mxo.Q4_K, mxo.Q5_K, mxo.Q6_K, mxo.Q8_0, mxo.Q5_0, mxo.F16, mxo.F32])
def test_matmul_vs_float64_brute_force(t):
    rng = np.random.default_rng(t)
    k, n = 512, 33
    w = mxo.quantize(t, rng.standard_normal((n, k)).astype(np.float32) * 0.02)
    a = rng.standard_normal((2, k)).astype(np.float32)
    wd = mxo.dequant(t, w, n, k).astype(np.float64)
    want = a.astype(np.float64) @ wd.T
    got = mxo.matmul_rhs_t(t, a, w, n)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6 * np.abs(want).max())


# ---- layer ops -------------------------------------------------------------------

def test_rmsnorm_vs_reference_vectors():
    x, y = VEC["rms_x"], VEC["rms_y"]
    for r in range(x.shape[0]):
        assert same_bits(mxo.rmsnorm(x[r], None, 1e-6), y[r])


def test_rmsnorm_closed_form():
    x = np.array([3.0, 4.0], np.float32)
    # mean square 12.5 -> y = x / sqrt(12.5 + eps)
    y = mxo.rmsnorm(x, np.array([2.0, 0.5], np.float32), 0.0)
    np.testing.assert_allclose(y, [2 * 3 / np.sqrt(12.5), 0.5 * 4 / np.sqrt(12.5)], rtol=1e-7)


@pytest.mark.parametrize("neox", [0, 1])
def test_rope_vs_reference_vectors(neox):
    x, ys = VEC[f"rope{neox}_x"], VEC[f"rope{neox}_y"]
    for pos, y in zip((0, 1, 7, 1000, 8191), ys):
        assert same_bits(mxo.rope(x, 8, 128, pos, 1e6, bool(neox)), y)


def test_rope_invariants():
    rng = np.random.default_rng(5)
    x = rng.standard_normal(4 * 64).astype(np.float32)
    assert np.array_equal(mxo.rope(x, 4, 64, 0, 1e6), x)           # position 0 is the identity
    for neox in (False, True):
        y = mxo.rope(x, 4, 64, 123, 1e4, neox)                       # rotations preserve pair norms
        half = 32
        for h in range(4):
            a = x[h * 64:(h + 1) * 64].astype(np.float64)
            b = y[h * 64:(h + 1) * 64].astype(np.float64)
            pa = (a[:half], a[half:]) if neox else (a[0::2], a[1::2])
            pb = (b[:half], b[half:]) if neox else (b[0::2], b[1::2])
            np.testing.assert_allclose(pa[0] ** 2 + pa[1] ** 2, pb[0] ** 2 + pb[1] ** 2, rtol=1e-5)
    # pair 0 rotates by exactly `pos` radians (inv_freq = 1)
    v = np.zeros(64, np.float32)
    v[0] = 1.0
    y = mxo.rope(v, 1, 64, 3, 1e4)
    np.testing.assert_allclose(y[:2], [np.cos(3.0), np.sin(3.0)], rtol=1e-6)


def test_softmax_vs_reference_vectors():
    assert same_bits(mxo.softmax(VEC["sm_x"]), VEC["sm_y"])


def test_softmax_closed_form():
    y = mxo.softmax(np.log(np.array([1, 2, 3, 4], np.float32)))
    np.testing.assert_allclose(y, [0.1, 0.2, 0.3, 0.4], rtol=1e-6)


def test_sampler_greedy_and_seeded():
    rng = np.random.default_rng(9)
    logits = rng.standard_normal(1000).astype(np.float32)
    tok, _ = mxo.sample(logits, 1, 0.0, 1.0, 0.0, 123)
    assert tok == int(np.argmax(logits))
    # top-k draw stays in the top k and is reproducible from the seed
    seen = []
    st = 42
    for _ in range(200):
        tok, st = mxo.sample(logits, 8, 0.8, 1.0, 0.0, st)
        seen.append(tok)
    top8 = set(np.argsort(-logits)[:8].tolist())
    assert set(seen) <= top8 and len(set(seen)) > 1
    st2, again = 42, []
    for _ in range(200):
        tok, st2 = mxo.sample(logits, 8, 0.8, 1.0, 0.0, st2)
        again.append(tok)
    assert seen == again
    # frequencies follow softmax(l / T) over the top 8
    big = []
    st = 7
    for _ in range(20000):
        tok, st = mxo.sample(logits, 8, 0.8, 1.0, 0.0, st)
        big.append(tok)
    ids = np.argsort(-logits)[:8]
    p = np.exp((logits[ids] - logits[ids].max()) / 0.8)
    p /= p.sum()
    freq = np.array([big.count(int(i)) for i in ids]) / len(big)
    np.testing.assert_allclose(freq, p, atol=0.015)
