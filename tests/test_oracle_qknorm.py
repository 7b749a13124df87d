"""Independent pins of oracle functions that neither the reference's tests
nor its compiled code check: Qwen3 QK-norm placement in the model step, the
top-p / min-p cuts of the sampler, and the logit edits before the choice
(CPU only).

QK-norm.  The reference layer goes projection -> bias -> RoPE
(src/transformer/transformer.cpp:406-514) and never loads attn_{q,k}_norm.
The Qwen3 architecture applies a per-head RMSNorm with a [head_dim] weight to
q and k after the projections and before RoPE.  A float64 numpy forward of a
tiny Qwen3 model with F32 weights, written here from that definition and not
from the oracle's code, must reproduce the oracle's per-layer hidden states.
The norm weights of the synthetic model are not uniform, so the norm does
not commute with the RoPE rotation: placing it after RoPE, swapping the q
and k weights, or dropping it all fail the comparison (checked below on the
numpy side).  The synthetic models carry no biases (Qwen3 has none), so the
order of bias and norm is not exercised.

Sampler.  minxfmr.cpp:2091-2171: softmax over the top k at temperature T,
then the top-p prefix (first i with cumulative p >= top_p) renormalised,
then the min-p prefix (p >= min_p * p_max) renormalised, then a draw.  With
logits log(p) for chosen p the kept set and its probabilities are known in
closed form; no draw may leave the set and 20k-draw frequencies must match.

Logit edits.  minxfmr.cpp:2047-2089: suppressed ids to -inf, then per
distinct id of the last N history ids (count c):
l <- (l <= 0 ? l * rp : l / rp) - c * fp - presence.  Checked on values
worked by hand, including the window, the zero-logit branch and the
neutral / empty-window cases.
"""
from __future__ import annotations

import numpy as np
import pytest

import gguf_synth
import mxo

ARCH = dict(name="qwen3", n_layer=2, n_embd=128, n_head=4, n_head_kv=2, head_dim=32, n_ff=256, n_vocab=64,
            qk_norm=True, tied=False, wtype=mxo.F32, out_type=mxo.F32, embd_type=mxo.F32, rope_theta=1e4,
            eps=1e-6)
TOKENS = [3, 17, 63, 0, 42, 42, 7, 5]


def f64(keep, name, rows=None, cols=None):
    t, ne, raw = keep[name]
    assert t == mxo.F32
    v = raw.view(np.float32).astype(np.float64)
    return v.reshape(ne[1], ne[0]) if len(ne) == 2 else v


def rms(x, w, eps):
    return x / np.sqrt(np.mean(x * x) + eps) * w


def rope_pairs(v, pos, theta):
    """Adjacent pairs (2i, 2i+1) of each head rotate by pos * theta^(-2i/d)."""
    d = v.shape[-1]
    ang = pos * theta ** (-np.arange(0, d, 2) / d)
    c, s = np.cos(ang), np.sin(ang)
    a, b = v[..., 0::2].copy(), v[..., 1::2].copy()
    out = np.empty_like(v)
    out[..., 0::2] = a * c - b * s
    out[..., 1::2] = a * s + b * c
    return out


def numpy_forward(keep, arch, tokens, mode="qwen3"):
    """Per-token, per-layer hidden states of the decoder stack in float64.
    mode: "qwen3" (norm before RoPE), "after_rope", "swapped" (q uses the k
    weight and back), "none" (no QK-norm)."""
    nl, d, nh, nkv, hd = arch["n_layer"], arch["n_embd"], arch["n_head"], arch["n_head_kv"], arch["head_dim"]
    eps, theta = arch["eps"], arch["rope_theta"]
    emb = f64(keep, "token_embd.weight")
    L = [{r: f64(keep, f"blk.{l}.{r}.weight") for r in
          ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_q_norm", "attn_k_norm", "attn_output", "ffn_norm",
           "ffn_gate", "ffn_up", "ffn_down")} for l in range(nl)]
    kc = [[] for _ in range(nl)]
    vc = [[] for _ in range(nl)]
    out = []
    for pos, tok in enumerate(tokens):
        x = emb[tok].copy()
        per = []
        for l in range(nl):
            W = L[l]
            xn = rms(x, W["attn_norm"], eps)
            q = (W["attn_q"] @ xn).reshape(nh, hd)
            k = (W["attn_k"] @ xn).reshape(nkv, hd)
            v = (W["attn_v"] @ xn).reshape(nkv, hd)
            qw, kw = W["attn_q_norm"], W["attn_k_norm"]
            if mode == "swapped":
                qw, kw = kw, qw
            norm = lambda m, w: np.stack([rms(r, w, eps) for r in m])
            if mode in ("qwen3", "swapped"):
                q, k = norm(q, qw), norm(k, kw)
            q, k = rope_pairs(q, pos, theta), rope_pairs(k, pos, theta)
            if mode == "after_rope":
                q, k = norm(q, qw), norm(k, kw)
            kc[l].append(k)
            vc[l].append(v)
            K, V = np.stack(kc[l]), np.stack(vc[l])  # [pos+1][nkv][hd]
            att = np.empty((nh, hd))
            for h in range(nh):
                g = h // (nh // nkv)
                s = K[:, g, :] @ q[h] / np.sqrt(hd)
                p = np.exp(s - s.max())
                p /= p.sum()
                att[h] = p @ V[:, g, :]
            x = x + W["attn_output"] @ att.reshape(-1)
            xn = rms(x, W["ffn_norm"], eps)
            gt, up = W["ffn_gate"] @ xn, W["ffn_up"] @ xn
            x = x + W["ffn_down"] @ (gt / (1.0 + np.exp(-gt)) * up)
            per.append(x.copy())
        out.append(np.stack(per))
    return np.stack(out)


def oracle_trace(path, flags=0):
    m = mxo.Model(path, n_ctx=64, flags=flags, threads=1)
    out = []
    for t in TOKENS:
        _, tr = m.step(t, want_logits=False, trace=True)
        out.append(tr[:-1].astype(np.float64))
    m.close()
    return np.stack(out)


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    keep = {}
    p = gguf_synth.build(tmp_path_factory.mktemp("qk") / "qk.gguf", gguf_synth.Arch(**ARCH), seed=77, keep=keep)
    return p, keep


def test_qk_norm_placement_matches_float64_forward(model):
    p, keep = model
    got = oracle_trace(p)
    want = numpy_forward(keep, ARCH, TOKENS)
    scale = np.abs(want).max()
    err = np.abs(got - want).max() / scale
    assert err < 1e-5, err
    # the comparison can tell the placements apart
    for mode in ("after_rope", "swapped", "none"):
        alt = numpy_forward(keep, ARCH, TOKENS, mode)
        assert np.abs(alt - want).max() / scale > 100 * max(err, 1e-7), mode


def test_no_qk_norm_flag_matches_float64_forward_without_norm(model):
    p, keep = model
    got = oracle_trace(p, mxo.OPEN_NO_QK_NORM)
    want = numpy_forward(keep, ARCH, TOKENS, "none")
    assert np.abs(got - want).max() / np.abs(want).max() < 1e-5


# ---- top-p / min-p --------------------------------------------------------

def draws(logits, top_k, temp, top_p, min_p, n, seed):
    out, st = [], seed
    for _ in range(n):
        tok, st = mxo.sample(logits, top_k, temp, top_p, min_p, st)
        out.append(tok)
    return np.array(out)


P4 = np.array([0.4, 0.3, 0.2, 0.1])
# (temperature, top_p, min_p) -> the kept ids (of the four) and their probabilities
CASES = [
    ((1.0, 0.65, 0.0), [4 / 7, 3 / 7]),          # 0.4 < 0.65 <= 0.7: two kept
    ((1.0, 0.75, 0.0), [4 / 9, 3 / 9, 2 / 9]),    # 0.7 < 0.75 <= 0.9: three
    ((1.0, 1.0, 0.6), [4 / 7, 3 / 7]),            # p >= 0.24: 0.4, 0.3
    ((1.0, 0.95, 0.3), [4 / 9, 3 / 9, 2 / 9]),    # top-p keeps four, min-p (>= 0.12) three
    ((0.5, 0.8, 0.0), [16 / 25, 9 / 25]),         # T = 0.5 squares p: .533, .3, .133, .033
    ((1.0, 1.5, 0.0), [0.4, 0.3, 0.2, 0.1]),      # top_p above 1 means 1
    ((1.0, -1.0, 0.0), [0.4, 0.3, 0.2, 0.1]),     # top_p <= 0 means 1
    ((1.0, 1.0, 2.0), [1.0]),                     # min_p clamped to 1: only the maximum
]


@pytest.mark.parametrize("params,probs", CASES, ids=[f"T{a}-p{b}-m{c}" for (a, b, c), _ in CASES])
def test_sampler_top_p_min_p_closed_form(params, probs):
    temp, top_p, min_p = params
    rng = np.random.default_rng(1)
    n = 50
    ids = rng.permutation(n)[:4]          # the four candidates at scattered ids
    logits = np.full(n, -40.0)
    logits[ids] = np.log(P4)
    logits = logits.astype(np.float32)
    got = draws(logits, 6, temp, top_p, min_p, 20000, 99)   # top_k 6 admits two -40 logits (p ~ 1e-17)
    kept = ids[:len(probs)]
    assert set(got.tolist()) <= set(kept.tolist()), set(got.tolist()) - set(kept.tolist())
    freq = np.array([(got == i).mean() for i in kept])
    np.testing.assert_allclose(freq, probs, atol=0.015)


# ---- logit edits before the choice (minxfmr.cpp:2047-2089) -------------------

def test_logit_edits_closed_form():
    """Values worked by hand from the reference's formula:
    l <- (l <= 0 ? l * rp : l / rp) - count * fp - presence, once per distinct
    id of the last N history ids; suppressed ids to -inf."""
    lg = np.array([2.0, -1.0, 0.5, 3.0, 1.0], np.float32)
    hist = [0, 0, 1, 3]
    got = mxo.logit_edits(lg, hist, (), -1, 2.0, 0.5, 1.0)
    # id 0 twice: 2/2 - 1 - 1; id 1 once: -1*2 - 0.5 - 1; id 3 once: 3/2 - 0.5 - 1
    np.testing.assert_array_equal(got, np.array([-1.0, -3.5, 0.5, 0.0, 1.0], np.float32))
    # window of the last two ids: 1 and 3 only
    got = mxo.logit_edits(lg, hist, (), 2, 2.0, 0.5, 1.0)
    np.testing.assert_array_equal(got, np.array([2.0, -3.5, 0.5, 0.0, 1.0], np.float32))
    # suppression, and a zero logit takes the multiplying branch
    z = np.array([0.0, 1.0, 1.0], np.float32)
    got = mxo.logit_edits(z, [0, 0], [2], -1, 3.0, 0.25, 0.0)
    np.testing.assert_array_equal(got, np.array([-0.5, 1.0, -np.inf], np.float32))
    # neutral penalties change nothing, repeat alone divides / multiplies
    np.testing.assert_array_equal(mxo.logit_edits(lg, hist, (), -1, 1.0, 0.0, 0.0), lg)
    got = mxo.logit_edits(lg, hist, (), -1, 1.5, 0.0, 0.0)
    np.testing.assert_allclose(got, [2.0 / 1.5, -1.5, 0.5, 2.0, 1.0], rtol=1e-7)
    # an empty window (N = 0) skips the penalty pass but not suppression
    got = mxo.logit_edits(lg, hist, [1], 0, 2.0, 0.5, 1.0)
    np.testing.assert_array_equal(got, np.array([2.0, -np.inf, 0.5, 3.0, 1.0], np.float32))
