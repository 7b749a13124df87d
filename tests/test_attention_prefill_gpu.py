"""Prefill attention on the matrix cores (GPU): mxh_attention_prefill.

For each of m prompt tokens at positions p0 .. p0+m-1 and each q head, the
reference (transformer.cpp:529-629) takes softmax(q.k / sqrt(hd)) over cache
positions 0 .. pos and sums the V rows with those weights.  The expected
values here are that computation in float64 on exactly the fp16 K/V values
the kernel reads.  The kernel keeps q and the probabilities as fp16 hi + lo
pairs (about 22 significant bits) with fp32 accumulation, so the admitted
error is |err| <= 1e-4 * max|V| + 1e-4 * |want|.

Cache rows past p0+m hold NaN and the output buffer starts as NaN: a read
past the causal limit or an output left unwritten fails the check.
"""
from __future__ import annotations

import numpy as np
import pytest

import mxhip

pytestmark = pytest.mark.gpu

# (nh, nkv, hd, p0, m): GQA groups 1, 2, 3, 4, 8; first chunk, later chunks,
# chunk lengths that leave partial query tiles and partial key stages
CASES = [
    (32, 8, 128, 0, 512),
    (32, 8, 128, 3000, 512),
    (32, 8, 128, 70, 1),
    (16, 8, 64, 0, 70),
    (16, 8, 64, 511, 130),
    (6, 2, 64, 100, 45),
    (8, 1, 32, 0, 33),
    (8, 1, 32, 1000, 200),
    (2, 2, 128, 63, 65),
]


def reference(q, kc, vc, p0, m, nh, nkv, hd):
    """float64 causal attention of rows p0 .. p0+m-1."""
    group = nh // nkv
    L = p0 + m
    qf = q.astype(np.float64).reshape(m, nh, hd)
    kf = kc[:L].astype(np.float64).reshape(L, nkv, hd)
    vf = vc[:L].astype(np.float64).reshape(L, nkv, hd)
    out = np.empty((m, nh, hd))
    pos = p0 + np.arange(m)
    mask = np.arange(L)[None, :] > pos[:, None]  # [m][L]
    for hq in range(nh):
        g = hq // group
        s = (qf[:, hq, :] @ kf[:, g, :].T) / np.sqrt(hd)
        s[mask] = -np.inf
        s -= s.max(axis=1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=1, keepdims=True)
        out[:, hq, :] = p @ vf[:, g, :]
    return out.reshape(m, nh * hd)


@pytest.mark.parametrize("nh,nkv,hd,p0,m", CASES, ids=[f"h{a}-kv{b}-d{c}-p{d}-m{e}" for a, b, c, d, e in CASES])
def test_attention_prefill_matches_float64(mxh, nh, nkv, hd, p0, m):
    rng = np.random.default_rng(nh * 1000 + hd * 10 + p0 + m)
    n_ctx = p0 + m + 40
    q = (rng.standard_normal((m, nh * hd)) * 1.5).astype(np.float32)
    kc = rng.standard_normal((n_ctx, nkv * hd)).astype(np.float16)
    vc = rng.standard_normal((n_ctx, nkv * hd)).astype(np.float16)
    kc[p0 + m:] = np.float16(np.nan)
    vc[p0 + m:] = np.float16(np.nan)
    dq, dk, dv = (mxhip.DeviceBuffer.from_array(a) for a in (q, kc, vc))
    att = mxhip.DeviceBuffer.from_array(np.full(m * nh * hd, np.nan, np.float32))
    mxhip.attention_prefill(dq, dk, dv, att, p0, m, nh, nkv, hd)
    got = att.download(np.float32, m * nh * hd).reshape(m, nh * hd).astype(np.float64)
    want = reference(q, kc, vc, p0, m, nh, nkv, hd)
    vmax = float(np.abs(vc[: p0 + m].astype(np.float64)).max())
    bound = 1e-4 * vmax + 1e-4 * np.abs(want)
    err = np.abs(got - want)
    assert np.all(np.isfinite(got)), "non-finite output"
    assert np.all(err <= bound), f"worst {float((err / bound).max()):.3g} x bound at {np.unravel_index(np.argmax(err / bound), err.shape)}"
    for b in (dq, dk, dv, att):
        b.close()


def test_attention_prefill_rejects_bad_shapes(mxh):
    b = mxhip.DeviceBuffer(4096)
    with pytest.raises(mxhip.MxhError, match="unsupported"):
        mxhip.attention_prefill(b, b, b, b, 0, 1, 32, 8, 96)  # head_dim 96
    with pytest.raises(mxhip.MxhError, match="unsupported"):
        mxhip.attention_prefill(b, b, b, b, 0, 1, 36, 4, 128)  # 9 q heads per kv head
    with pytest.raises(mxhip.MxhError, match="unsupported"):
        mxhip.attention_prefill(b, b, b, b, 0, 0, 32, 8, 128)  # no tokens
    b.close()
