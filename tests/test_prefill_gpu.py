"""Batched prefill on the matrix cores (GPU).

The single-product GEMM entry (mxh_gemm_q_bf16) takes bf16 inputs: A rounded to bf16, the weights dequantized
exactly (the bit-exact decoder) and then rounded to bf16, products summed in
fp32.  Its reference here is the float64 product of exactly those bf16
values, so the only admitted difference is fp32 summation:
|err| <= 1e-5 * sum_k |a_k w_k| per output.

The exact-weight entry (mxh_gemm_q_f16, the model's prefill GEMM for
quantized rows) multiplies the weights' integer codes exactly and carries A
as fp16 hi + lo of a 2^e (about 22 significant bits); its reference is the
float64 product of the unrounded a with the exactly dequantized weights,
within 2^-19 * sum_k |a_k w_k| (22-bit inputs and fp32 sums), far below a
bf16-rounded weight's 2^-9.  The model's prefill is also checked end to end
against the token-by-token oracle.
"""
from __future__ import annotations

import numpy as np
import pytest

import mxhip
import mxo

pytestmark = pytest.mark.gpu

TYPES = {"Q4_K": mxo.Q4_K, "Q5_K": mxo.Q5_K, "Q8_0": mxo.Q8_0, "Q5_0": mxo.Q5_0, "F32": mxo.F32}


def bf16_round(a: np.ndarray) -> np.ndarray:
    """Round float32 to the nearest bf16 (ties to even), returned as float32."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


GEMM_CASES = [
    ("Q4_K", 1, 256, 256), ("Q4_K", 128, 128, 256), ("Q4_K", 300, 520, 512), ("Q4_K", 512, 1024, 4096),
    ("Q5_K", 77, 384, 512), ("Q8_0", 130, 200, 192), ("Q5_0", 64, 96, 128), ("F32", 33, 130, 64),
]


@pytest.mark.parametrize("name,m,n,k", GEMM_CASES, ids=[f"{a}-{b}x{c}x{d}" for a, b, c, d in GEMM_CASES])
def test_gemm_bf16_vs_rounded_reference(mxh, name, m, n, k):
    t = TYPES[name]
    rng = np.random.default_rng(m * 7 + n * 13 + k)
    wf = rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)
    w = mxo.quantize(t, wf)
    a = rng.standard_normal((m, k), dtype=np.float32)
    forms = (mxo.FORM_REF, mxo.FORM_GGML) if t in (mxo.Q4_K, mxo.Q5_K) else (mxo.FORM_REF,)
    dw = mxhip.DeviceBuffer.from_array(w)
    da = mxhip.DeviceBuffer.from_array(a)
    out = mxhip.DeviceBuffer(4 * m * n)
    for form in forms:
        wd = bf16_round(mxo.dequant(t, w, n, k, form)).astype(np.float64)
        ab = bf16_round(a).astype(np.float64)
        want = ab @ wd.T
        bound = 1e-5 * (np.abs(ab) @ np.abs(wd).T) + 1e-30
        mxhip.gemm_bf16(t, da, m, dw, n, k, out, form)
        got = out.download(np.float32, m * n).reshape(m, n).astype(np.float64)
        err = np.abs(got - want)
        assert np.all(err <= bound), f"form {form}: worst {float((err / bound).max()):.3g} x bound"
    for b in (dw, da, out):
        b.close()


F16_CASES = [
    ("Q4_K", 1, 256, 256), ("Q4_K", 128, 128, 256), ("Q4_K", 300, 520, 512), ("Q4_K", 512, 1024, 4096),
    ("Q5_K", 77, 384, 512), ("Q5_K", 200, 640, 1024), ("Q8_0", 130, 200, 256), ("Q8_0", 257, 300, 1024),
    ("Q5_0", 64, 96, 256), ("Q5_0", 9, 130, 512),
]


@pytest.mark.parametrize("name,m,n,k", F16_CASES, ids=[f"{a}-{b}x{c}x{d}" for a, b, c, d in F16_CASES])
@pytest.mark.parametrize("tiled", [False, True], ids=["gguf", "tiled"])
def test_gemm_f16_exact_weights(mxh, name, m, n, k, tiled):
    t = TYPES[name]
    rng = np.random.default_rng(m * 5 + n * 11 + k)
    w = mxo.quantize(t, rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    a = rng.standard_normal((m, k), dtype=np.float32)
    a[:, 5] *= 1e-3  # small and large elements in one row
    forms = (mxo.FORM_REF, mxo.FORM_GGML) if t in (mxo.Q4_K, mxo.Q5_K) else (mxo.FORM_REF,)
    dw = mxhip.DeviceBuffer.from_array(w)
    tt = mxhip.tile_rows(t, dw, n, k) if tiled else t
    da = mxhip.DeviceBuffer.from_array(a)
    out = mxhip.DeviceBuffer(4 * m * n)
    for form in forms:
        wd = mxo.dequant(t, w, n, k, form).astype(np.float64)
        want = a.astype(np.float64) @ wd.T
        bound = 2.0 ** -19 * (np.abs(a).astype(np.float64) @ np.abs(wd).T) + 1e-30
        mxhip.gemm_f16(tt, da, m, dw, n, k, out, form)
        got = out.download(np.float32, m * n).reshape(m, n).astype(np.float64)
        err = np.abs(got - want)
        assert np.all(err <= bound), f"form {form}: worst {float((err / bound).max()):.3g} x bound"
    for b in (dw, da, out):
        b.close()


def test_gemm_f16_rejects_bad_shapes(mxh):
    dw = mxhip.DeviceBuffer(1 << 16)
    da = mxhip.DeviceBuffer(1 << 16)
    with pytest.raises(mxhip.MxhError, match="bad shape"):
        mxhip.gemm_f16(mxo.Q8_0, da, 1, dw, 1, 96, da)  # k not a multiple of 256
    with pytest.raises(mxhip.MxhError, match="bad shape"):
        mxhip.gemm_f16(mxo.F32, da, 1, dw, 1, 256, da)  # no integer codes


def test_gemm_bf16_rejects_bad_shapes(mxh):
    dw = mxhip.DeviceBuffer(4096)
    da = mxhip.DeviceBuffer(4096)
    with pytest.raises(mxhip.MxhError, match="bad shape"):
        mxhip.gemm_bf16(mxo.Q8_0, da, 1, dw, 1, 32, da)  # k not a multiple of 64
    with pytest.raises(mxhip.MxhError, match="bad shape"):
        mxhip.gemm_bf16(mxo.Q4_K, da, 1, dw, 1, 64, da)  # k not a multiple of 256 for Q4_K


# ---- batched prefill through the model --------------------------------------

from test_model_gpu import TINY, VARIANTS, build, close_enough  # noqa: E402


@pytest.mark.parametrize("name", list(VARIANTS))
@pytest.mark.parametrize("n_ctx,n_prompt", [(128, 70), (600, 530)])
@pytest.mark.parametrize("flags", [0, mxhip.MODEL_BF16_PREFILL], ids=["default", "bf16split"])
def test_batched_prefill_then_step(mxh, tmp_path, name, n_ctx, n_prompt, flags):
    """Prompt fed through the matrix-core prefill (one chunk of 70, or 512 +
    18), then one decode step: its per-layer hidden states and logits are
    within the parity bar of the oracle run token by token (fp16 cache).
    Default: quantized projections on the exact-weight fp16 GEMM, F32 ones
    split bf16; MODEL_BF16_PREFILL: every projection split bf16."""
    prefill_vs_oracle(tmp_path, name, n_ctx, n_prompt, flags)


def test_batched_prefill_wide_tiles(mxh, tmp_path):
    """Projections of at least 2048 rows with more than 128 prompt rows take
    the Q4_K GEMM's 256-row weight tiles (8 waves per workgroup); the tiny
    shapes above take the 128-row tiles.  Hidden size 2048 puts q|k|v, o,
    gate|up and down on the wide tiles."""
    prefill_vs_oracle(tmp_path, "q4k-qknorm", 600, 530, 0, n_embd=2048, n_head=16, n_head_kv=4, head_dim=128,
                      n_ff=2048)


def prefill_vs_oracle(tmp_path, name, n_ctx, n_prompt, flags, **over):
    p = build(tmp_path, name, **over)
    rng = np.random.default_rng(17)
    prompt = rng.integers(0, TINY["n_vocab"], n_prompt).astype(np.int32)
    nxt = int(rng.integers(0, TINY["n_vocab"]))
    gm = mxhip.Model(p, n_ctx, flags)
    gm.prefill(prompt)
    lg, tr = gm.step(nxt, trace=True)
    om = mxo.Model(p, n_ctx, mxo.OPEN_KV_FP16)
    for t in prompt:
        om.step(int(t), want_logits=False)
    olg, otr = om.step(nxt, trace=True)
    ok, e1 = close_enough(tr, otr)
    assert ok, f"hidden trace error {e1}"
    ok, e2 = close_enough(lg, olg)
    assert ok, f"logits error {e2}"
    # split operands keep 16 (bf16) to 22 (fp16) bits: far inside the bar, as the fp32 path
    worst = max(e1 / max(1.0, float(np.abs(otr).max())), e2)
    assert worst < 1e-3, worst
    gm.close()


def test_token_prefill_flag_matches_oracle_exactly_as_decode(mxh, tmp_path):
    """MXH_MODEL_TOKEN_PREFILL keeps the fp32 GEMV path for the prompt."""
    p = build(tmp_path, "q4k-qknorm")
    prompt = np.random.default_rng(2).integers(0, TINY["n_vocab"], 20).astype(np.int32)
    a = mxhip.Model(p, 64, mxhip.MODEL_TOKEN_PREFILL)
    b = mxhip.Model(p, 64, mxhip.MODEL_TOKEN_PREFILL | mxhip.MODEL_NO_GRAPH)
    a.prefill(prompt)
    for t in prompt:
        b.step(int(t), logits=False)
    la, _ = a.step(3)
    lb, _ = b.step(3)
    assert np.array_equal(la, lb)
    a.close()
    b.close()
