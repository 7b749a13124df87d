"""Tiled device layout of the projection weights (GPU).

The model regroups the bytes of each Q4_K / Q8_0 weight row in HBM so that a
wave's 16-byte loads read whole cache lines; the arithmetic on the bytes is
unchanged.  Opening the same file with MXH_MODEL_GGUF_LAYOUT keeps the GGUF
block order, and both must give bit-identical logits and greedy ids, through
the batched prefill (matrix-core GEMM) and the decode step (GEMV), including
rows whose last tile is partial (K = 4608: 18 Q4_K blocks, tiles of 16 and 2;
Q5_K tiles of 8, 8 and 2; K = 6144: 24 Q6_K blocks, tiles of 16 and 8).
"""
from __future__ import annotations

import numpy as np
import pytest

import mxhip

pytestmark = pytest.mark.gpu

BASE = dict(n_layer=2, n_embd=256, n_head=4, n_head_kv=2, head_dim=64, n_ff=512, n_vocab=300)
CASES = {
    "q4k": dict(wtype=mxhip.Q4_K, out_type=mxhip.Q8_0, embd_type=mxhip.Q8_0, qk_norm=True),
    "q8-tied": dict(wtype=mxhip.Q8_0, out_type=mxhip.Q8_0, embd_type=mxhip.Q8_0, qk_norm=True, tied=True),
    "q4k-mixed-q5k": dict(wtype=mxhip.Q4_K, out_type=mxhip.Q8_0, embd_type=mxhip.Q4_K, qk_norm=False,
                          attn_v_type=mxhip.Q5_K, ffn_down_type=mxhip.Q5_K, arch="llama", rope_theta=5e5),
    "q4k-partial-tiles": dict(wtype=mxhip.Q4_K, out_type=mxhip.Q8_0, embd_type=mxhip.Q8_0, qk_norm=True,
                              n_embd=512, n_ff=4608, head_dim=128),
    # Q5_K down projection with K = 4608: 18 blocks, tiles of 8, 8 and 2
    "q5k-partial-tiles": dict(wtype=mxhip.Q4_K, out_type=mxhip.Q8_0, embd_type=mxhip.Q4_K, qk_norm=False,
                              attn_v_type=mxhip.Q5_K, ffn_down_type=mxhip.Q5_K, arch="llama", rope_theta=5e5,
                              n_embd=512, n_ff=4608, head_dim=128),
    # Q4_K_M mix with tiled Q6_K: head and attn_v at K = 2048 (one 16-block
    # tile), ffn_down at K = 6144 (tiles of 16 and 8)
    "q6k-partial-tiles": dict(wtype=mxhip.Q4_K, out_type=mxhip.Q6_K, embd_type=mxhip.Q4_K, qk_norm=False,
                              attn_v_type=mxhip.Q6_K, ffn_down_type=mxhip.Q6_K, arch="llama", rope_theta=5e5,
                              n_embd=2048, n_head=16, n_head_kv=4, n_ff=6144, head_dim=128),
}


def build(tmp_path, name):
    kw = dict(BASE)
    kw.update(CASES[name])
    arch = kw.pop("arch", "qwen3")
    p = tmp_path / f"{name}.gguf"
    mxhip.write_synthetic_gguf(p, arch, seed=23, **kw)
    return p


@pytest.mark.parametrize("name", list(CASES))
def test_tiled_layout_is_bit_identical(mxh, tmp_path, name):
    p = build(tmp_path, name)
    prompt = np.random.default_rng(3).integers(0, BASE["n_vocab"], 20).astype(np.int32)
    tiled = mxhip.Model(p, 96)
    gguf = mxhip.Model(p, 96, mxhip.MODEL_GGUF_LAYOUT)
    # batched prefill, then decode steps with logits
    for m in (tiled, gguf):
        m.prefill(prompt[:-1])
    for t in list(prompt[-1:]) + [7, 123, 42]:
        la, _ = tiled.step(int(t))
        lb, _ = gguf.step(int(t))
        assert np.array_equal(la, lb), f"logits differ after token {t}: max {np.abs(la - lb).max()}"
    # whole greedy generation (graphs, prefill and decode) from a reset
    ids_a, _, _ = tiled.generate(prompt, 24)
    ids_b, _, _ = gguf.generate(prompt, 24)
    assert np.array_equal(ids_a, ids_b)
