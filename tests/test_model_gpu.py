"""Device-resident decode step vs the CPU oracle (GPU).

Bars (north star): per-layer activations and logits within max-abs 2e-2 /
relative 1e-2 of the CPU backend; greedy ids identical for the first 64
generated tokens.  The oracle runs with an fp16-rounded KV cache for the
activation comparisons (the GPU cache is fp16); the greedy-token comparison
is made against both that oracle and the reference's fp32 cache.
"""
from __future__ import annotations

import warnings

import numpy as np
import pytest

import mxhip
import mxo

pytestmark = pytest.mark.gpu

TINY = dict(n_layer=3, n_embd=256, n_head=4, n_head_kv=2, head_dim=64, n_ff=512, n_vocab=300)
VARIANTS = {
    "q4k-qknorm": dict(wtype=mxhip.Q4_K, out_type=mxhip.Q8_0, embd_type=mxhip.Q8_0, qk_norm=True),
    "q8-tied": dict(wtype=mxhip.Q8_0, out_type=mxhip.Q8_0, embd_type=mxhip.Q8_0, qk_norm=True, tied=True),
    "q4k-mixed-q5k": dict(wtype=mxhip.Q4_K, out_type=mxhip.Q8_0, embd_type=mxhip.Q4_K, qk_norm=False,
                          attn_v_type=mxhip.Q5_K, ffn_down_type=mxhip.Q5_K, arch="llama", rope_theta=5e5),
    "q5_0-gqa8": dict(wtype=mxhip.Q5_0, out_type=mxhip.Q8_0, embd_type=mxhip.Q8_0, qk_norm=True, n_head=8,
                      n_head_kv=1, head_dim=32),
    "f32-hd128": dict(wtype=mxhip.F32, out_type=mxhip.F32, embd_type=mxhip.F32, n_head=2, n_head_kv=2, head_dim=128),
    # llama.cpp Q4_K_M mix: Q4_K projections, Q6_K head, attn_v and ffn_down
    # (here in the GGUF block order: K = 256 / 512), F16 embedding
    "q4k-m-q6k": dict(wtype=mxhip.Q4_K, out_type=mxhip.Q6_K, embd_type=mxhip.F16, attn_v_type=mxhip.Q6_K,
                      ffn_down_type=mxhip.Q6_K, qk_norm=False, arch="llama", rope_theta=5e5),
    "f16": dict(wtype=mxhip.F16, out_type=mxhip.F16, embd_type=mxhip.F16, qk_norm=True),
    # the Qwen3-8B attention shape: 4 q heads per kv head, head_dim 128
    "q4k-g4-hd128": dict(wtype=mxhip.Q4_K, out_type=mxhip.Q8_0, embd_type=mxhip.Q8_0, qk_norm=True, n_head=8,
                         n_head_kv=2, head_dim=128),
    # GGUF type 41 (one byte per element, the byte's value) for attn_v and
    # ffn_down, widened to F32 rows when the model opens
    "q4k-byte41": dict(wtype=mxhip.Q4_K, out_type=mxhip.Q8_0, embd_type=mxhip.Q8_0, qk_norm=True,
                       attn_v_type=mxhip.Q1_0, ffn_down_type=mxhip.Q1_0),
    # a type-41 token embedding, tied: the embedding rows and the lm-head
    # are the widened F32 rows
    "q8-tied-byte41": dict(wtype=mxhip.Q8_0, out_type=mxhip.Q8_0, embd_type=mxhip.Q1_0, qk_norm=True, tied=True),
}


def build(tmp_path, name, **over):
    kw = dict(TINY)
    kw.update(VARIANTS[name])
    kw.update(over)
    arch = kw.pop("arch", "qwen3")
    p = tmp_path / f"{name}.gguf"
    mxhip.write_synthetic_gguf(p, arch, seed=11, **kw)
    return p


def close_enough(got, want, atol=2e-2, rtol=1e-2):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    return bool(np.all(err <= atol + rtol * np.abs(want))), float(err.max())


@pytest.mark.parametrize("name", list(VARIANTS))
@pytest.mark.parametrize("flags", [0, mxhip.MODEL_ROPE_NEOX | mxhip.MODEL_GGML_FORM])
def test_per_layer_activations_and_logits(mxh, tmp_path, name, flags):
    p = build(tmp_path, name)
    oflags = mxo.OPEN_KV_FP16 | (mxo.OPEN_ROPE_NEOX if flags & mxhip.MODEL_ROPE_NEOX else 0) | \
        (mxo.OPEN_GGML_FORM if flags & mxhip.MODEL_GGML_FORM else 0)
    gm = mxhip.Model(p, 64, flags)
    om = mxo.Model(p, 64, oflags)
    rng = np.random.default_rng(3)
    worst = 0.0
    for step in range(20):
        tok = int(rng.integers(0, TINY["n_vocab"]))
        lg, tr = gm.step(tok, trace=True)
        olg, otr = om.step(tok, trace=True)
        ok, e1 = close_enough(tr, otr)
        assert ok, f"step {step}: hidden trace error {e1}"
        ok, e2 = close_enough(lg, olg)
        assert ok, f"step {step}: logits error {e2}"
        worst = max(worst, e1 / max(1.0, float(np.abs(otr).max())), e2)
    # much tighter than the bar: only summation order and fp32 rounding differ
    assert worst < 1e-3, worst
    gm.close()


@pytest.mark.parametrize("name,n_ctx,warm", [("q4k-qknorm", 600, 300), ("q5_0-gqa8", 1100, 300),
                                             ("q8-tied", 1100, 300), ("f32-hd128", 4000, 520),
                                             ("q4k-qknorm", 8200, 4150), ("q5_0-gqa8", 4200, 4100),
                                             ("f32-hd128", 4096, 600), ("q8-tied", 4500, 4480),
                                             ("q4k-g4-hd128", 600, 300), ("q4k-g4-hd128", 4400, 4380)])
def test_multi_split_attention(mxh, tmp_path, name, n_ctx, warm):
    """Contexts long enough for several attention splits per q head.
    Below 4096 positions of context the per-q-head kernel runs: the grid
    holds min(8, ceil(n_ctx / 256)) splits and a launch uses
    min(grid, ceil(L / 128)) of them; the rest leave empty partials that the
    merge must skip.  Checked at positions warm .. warm+5 (and 0 .. 2):
    3 of 3 splits (Q4_K o-projection merging in its x staging), 3 of 5
    (Q5_0 with hd 32 and 8 q heads per kv head; Q8_0 tied, the tiled
    two-row merge), 5 of 8 (F32 o-projection: the separate merge kernel).
    From 4096 the grouped kernel runs (one workgroup per kv head and split,
    the grid one workgroup per CU over the kv heads, at least 64 positions
    per active split, the merge kernel before the o-projection): hd 64 with
    2 q heads per kv head at L about 4150 (65 of 128 splits), hd 32 with 8
    q heads per kv head at L about 4100 (65 of 256), hd 128 with one q head
    per kv head at L about 600 (10 of 128, F32 rows), splits of 35
    positions near the end of a 4500-position context (all 128), and the
    Qwen3-8B shape (4 q heads per kv head, hd 128) on both kernels."""
    p = build(tmp_path, name)
    gm = mxhip.Model(p, n_ctx)
    om = mxo.Model(p, n_ctx, mxo.OPEN_KV_FP16)
    rng = np.random.default_rng(7)
    toks = rng.integers(0, TINY["n_vocab"], warm + 6)
    worst = 0.0
    for i, tok in enumerate(toks):
        check = i < 3 or i >= warm
        lg, tr = gm.step(int(tok), trace=check, logits=check)
        olg, otr = om.step(int(tok), trace=check)
        if not check:
            continue
        ok, e1 = close_enough(tr, otr)
        assert ok, f"position {i}: hidden trace error {e1}"
        ok, e2 = close_enough(lg, olg)
        assert ok, f"position {i}: logits error {e2}"
        worst = max(worst, e1 / max(1.0, float(np.abs(otr).max())), e2)
    assert worst < 1e-3, worst
    gm.close()


@pytest.mark.parametrize("name,n_ctx,n_steps", [("q4k-qknorm", 24, 70), ("q5_0-gqa8", 40, 100),
                                                ("q4k-g4-hd128", 300, 620), ("q4k-g4-hd128", 4096, 4125)])
def test_ring_past_full_cache(mxh, tmp_path, name, n_ctx, n_steps):
    """Past n_ctx tokens the cache is the reference's ring (kv_cache.cpp:50-75):
    each step attends the last n_ctx tokens and itself with RoPE at position
    n_ctx, and overwrites the oldest row.  Hidden states and logits against
    the oracle's ring, before the cache fills, across the wrap and after more
    than one full turn of the ring (two turns at 300), on the per-q-head
    kernel (1, 2 and 8 q heads per kv head; 2 splits at 300) and the grouped
    kernel (4096)."""
    p = build(tmp_path, name)
    gm = mxhip.Model(p, n_ctx)
    om = mxo.Model(p, n_ctx, mxo.OPEN_KV_FP16)
    toks = np.random.default_rng(11).integers(0, TINY["n_vocab"], n_steps)
    checks = set(range(3)) | set(range(n_ctx - 2, n_ctx + 4)) | set(range(n_steps - 4, n_steps))
    worst = 0.0
    for i, tok in enumerate(toks):
        check = i in checks
        lg, tr = gm.step(int(tok), trace=check, logits=check)
        olg, otr = om.step(int(tok), trace=check)
        if not check:
            continue
        ok, e1 = close_enough(tr, otr)
        assert ok, f"position {i}: hidden trace error {e1}"
        ok, e2 = close_enough(lg, olg)
        assert ok, f"position {i}: logits error {e2}"
        worst = max(worst, e1 / max(1.0, float(np.abs(otr).max())), e2)
    assert worst < 1e-3, worst
    gm.close()


@pytest.mark.parametrize("name,n_ctx", [("q4k-qknorm", 24), ("q4k-g4-hd128", 4096)])
def test_prompt_longer_than_cache(mxh, tmp_path, name, n_ctx):
    """A prompt longer than the cache: batched chunks up to n_ctx, then token
    steps on the ring.  The next step's logits match the oracle fed token by
    token, and greedy decoding from there (HIP graph) gives the ids of the
    step-by-step eager path."""
    p = build(tmp_path, name)
    n_prompt = n_ctx + min(n_ctx // 2, 40) + 5
    prompt = np.random.default_rng(12).integers(0, TINY["n_vocab"], n_prompt).astype(np.int32)
    gm = mxhip.Model(p, n_ctx)
    om = mxo.Model(p, n_ctx, mxo.OPEN_KV_FP16)
    gm.prefill(prompt[:-1])
    assert gm.position == n_prompt - 1
    for t in prompt[:-1]:
        om.step(int(t), trace=False)
    lg, _ = gm.step(int(prompt[-1]))
    olg, _ = om.step(int(prompt[-1]), trace=False)
    ok, err = close_enough(lg, olg)
    assert ok and err < 1e-3, f"logits after the prompt: error {err}"
    ids, _ = gm.decode(12)
    gm.close()
    em = mxhip.Model(p, n_ctx, mxhip.MODEL_NO_GRAPH | mxhip.MODEL_TOKEN_PREFILL)
    em.prefill(prompt[:-1])
    em.step(int(prompt[-1]))
    eids, _ = em.decode(12)
    em.close()
    assert ids.tolist() == eids.tolist()


@pytest.mark.parametrize("n_ctx", [128, 4200, 24])
def test_bench_attention_leaves_decoding_unchanged(mxh, tmp_path, n_ctx):
    """mxh_model_bench_attention reruns every layer's decode attention at the
    current position (the per-q-head kernel at 128 positions of context, the
    grouped kernel and its merge at 4200, the ring's kernels past a 24-row
    cache): its launch and byte counts follow the rows attended, and
    decoding afterwards gives the ids of an uninterrupted run (the cache row
    it rewrites is written again by the next step)."""
    p = build(tmp_path, "q4k-g4-hd128")
    prompt = np.random.default_rng(21).integers(0, TINY["n_vocab"], 30).astype(np.int32)
    a = mxhip.Model(p, n_ctx)
    ids_a, _, _ = a.generate(prompt, 8)
    rest_a, _ = a.decode(12)
    b = mxhip.Model(p, n_ctx)
    ids_b, _, _ = b.generate(prompt, 8)
    pos = b.position
    ms, n, nbytes = b.bench_attention(3)
    cfg = b.cfg
    assert n == 3 * cfg.n_layer
    assert nbytes == 3 * cfg.n_layer * 2 * min(pos, n_ctx) * cfg.n_head_kv * cfg.head_dim * 2
    assert ms > 0
    rest_b, _ = b.decode(12)
    assert np.array_equal(ids_a, ids_b)
    assert np.array_equal(rest_a, rest_b)
    a.close()
    b.close()


@pytest.mark.parametrize("name", ["q4k-qknorm", "q4k-mixed-q5k"])
def test_graph_generate_matches_eager_steps_and_oracle(mxh, tmp_path, name):
    p = build(tmp_path, name)
    prompt = np.random.default_rng(5).integers(0, TINY["n_vocab"], 12).astype(np.int32)
    gm = mxhip.Model(p, 128)
    ids, _, _ = gm.generate(prompt, 48)
    # eager path (no graphs) must give the same ids
    em = mxhip.Model(p, 128, mxhip.MODEL_NO_GRAPH)
    ids2, _, _ = em.generate(prompt, 48)
    assert np.array_equal(ids, ids2)
    # generating twice (reset) is reproducible
    ids3, _, _ = gm.generate(prompt, 48)
    assert np.array_equal(ids, ids3)
    # oracle with the reference fp32 cache
    om = mxo.Model(p, 128)
    want = []
    lg = None
    for t in prompt:
        lg, _ = om.step(int(t))
    for _ in range(48):
        nxt = mxo.lib.mxo_argmax(lg.ctypes.data, lg.size)
        want.append(nxt)
        lg, _ = om.step(nxt)
    assert ids.tolist() == want


def test_q4_k_m_tiled_q6k_vs_oracle(mxh, tmp_path):
    """A llama.cpp Q4_K_M-style mix at widths the tiled Q6_K layout takes
    (head and attn_v at K = 2048, ffn_down at K = 6144: tiles of 16 and 8
    blocks), F16 embedding: per-layer hidden states and logits within the
    bar (and 1e-3) over token steps, then 32 greedy ids from a batched
    prefill equal to the oracle's (fp16 cache)."""
    V = 1000
    p = build(tmp_path, "q4k-m-q6k", n_layer=2, n_embd=2048, n_head=16, n_head_kv=4, head_dim=128, n_ff=6144,
              n_vocab=V)
    gm = mxhip.Model(p, 128)
    om = mxo.Model(p, 128, mxo.OPEN_KV_FP16, threads=16)
    rng = np.random.default_rng(17)
    worst = 0.0
    for step in range(6):
        tok = int(rng.integers(0, V))
        lg, tr = gm.step(tok, trace=True)
        olg, otr = om.step(tok, trace=True)
        ok, e1 = close_enough(tr, otr)
        assert ok, f"step {step}: hidden trace error {e1}"
        ok, e2 = close_enough(lg, olg)
        assert ok, f"step {step}: logits error {e2}"
        worst = max(worst, e1 / max(1.0, float(np.abs(otr).max())), e2)
    assert worst < 1e-3, worst
    prompt = rng.integers(0, V, 24).astype(np.int32)
    ids, _, _ = gm.generate(prompt, 32)
    gm.close()
    om.reset()
    lg = None
    for t in prompt:
        lg, _ = om.step(int(t))
    for i in range(32):
        top = np.sort(lg)[-2:]
        want = int(np.argmax(lg))
        assert int(ids[i]) == want, f"step {i}: id {ids[i]} != oracle {want} (top-2 margin {top[1] - top[0]:.3g})"
        lg, _ = om.step(want)
    om.close()


@pytest.mark.parametrize("flags", [0, mxhip.MODEL_GGML_FORM], ids=["ref-form", "ggml-form"])
def test_qwen3_8b_widths_vs_oracle(mxh, tmp_path, flags):
    """Hidden size 4096, FFN 12288 and 32 / 8 heads of 128, the Qwen3-8B
    widths, at two layers: every Q4_K projection runs the form it runs in
    the 8B model (q|k|v twelve waves in one step with the fused norm, o
    eight waves merging the attention splits, gate|up twelve waves in four
    SwiGLU steps, down eight waves in three steps of K = 12288).  Per-layer
    hidden states and logits within the bar (and 1e-3) of the oracle over 8
    token steps, in both scale forms, then 16 greedy ids from a prompt equal
    to the oracle's."""
    V = 1000
    p = build(tmp_path, "q4k-qknorm", n_layer=2, n_embd=4096, n_head=32, n_head_kv=8, head_dim=128, n_ff=12288,
              n_vocab=V)
    gm = mxhip.Model(p, 128, flags)
    oflags = mxo.OPEN_KV_FP16 | (mxo.OPEN_GGML_FORM if flags & mxhip.MODEL_GGML_FORM else 0)
    om = mxo.Model(p, 128, oflags, threads=16)
    rng = np.random.default_rng(29)
    worst = 0.0
    for step in range(8):
        tok = int(rng.integers(0, V))
        lg, tr = gm.step(tok, trace=True)
        olg, otr = om.step(tok, trace=True)
        ok, e1 = close_enough(tr, otr)
        assert ok, f"step {step}: hidden trace error {e1}"
        ok, e2 = close_enough(lg, olg)
        assert ok, f"step {step}: logits error {e2}"
        worst = max(worst, e1 / max(1.0, float(np.abs(otr).max())), e2)
    assert worst < 1e-3, worst
    prompt = rng.integers(0, V, 12).astype(np.int32)
    ids, _, _ = gm.generate(prompt, 16)
    gm.close()
    om.reset()
    lg = None
    for t in prompt:
        lg, _ = om.step(int(t))
    for i in range(16):
        top = np.sort(lg)[-2:]
        want = int(np.argmax(lg))
        assert int(ids[i]) == want, f"step {i}: id {ids[i]} != oracle {want} (top-2 margin {top[1] - top[0]:.3g})"
        lg, _ = om.step(want)
    om.close()


SWAP_EDITS = dict(suppress=[7, 11], repeat_last_n=24, repeat_penalty=1.3, frequency_penalty=0.4, presence_penalty=2.0)


@pytest.mark.parametrize("host_steps", [1, 2], ids=["handover-at-swap", "handover-after-host-step"])
@pytest.mark.parametrize("sampled", [False, True], ids=["greedy", "topk8"])
def test_first_token_swap_then_device(mxh, tmp_path, sampled, host_steps):
    """The coarse-step protocol (the reference's first step on the host, then
    the device from the host's id on) against the oracle.

    Host phase (device edits off, greedy head): the device returns the head's
    raw logits; the host applies the reference's edits (minxfmr.cpp:2047-2089)
    and takes the runner-up of its order, as the reference's first-token swap
    does when order[0] is invisible (:2189-2205).  With host_steps=2 one more
    step runs on the host: the swapped id is the device's input and the host
    chooses again.  Then the hand-over: the same edits and sampling set on the
    device, mxh_model_set_token with the host's last id, and 16 device-chosen
    ids.  They equal the oracle's continuing from the same ids, whose
    penalties count the swapped id in the history (:2388)."""
    p = build(tmp_path, "q4k-qknorm")
    prompt = np.random.default_rng(31).integers(0, TINY["n_vocab"], 16).astype(np.int32)
    e = SWAP_EDITS
    k, temp, seed, n_dev = 8, 0.8, 99, 16

    def edit(lg, hist):
        return mxo.logit_edits(lg, hist, e["suppress"], e["repeat_last_n"], e["repeat_penalty"],
                               e["frequency_penalty"], e["presence_penalty"])

    # oracle: prompt, the swap, the host steps, then the device's choice rule
    om = mxo.Model(p, 128)
    lg = None
    for t in prompt:
        lg, _ = om.step(int(t))
    hist = prompt.tolist()
    want_host_logits, host_ids = [], []
    for s in range(host_steps):
        want_host_logits.append(lg)
        ed = edit(lg, hist)
        order = np.argsort(-ed.astype(np.float64), kind="stable")
        nxt = int(order[1]) if s == 0 else int(order[0])
        host_ids.append(nxt)
        hist.append(nxt)
        lg, _ = om.step(nxt)
    want, state = [], seed
    for _ in range(n_dev):
        ed = edit(lg, hist)
        if sampled:
            nxt, state = mxo.sample(ed, k, temp, 1.0, 0.0, state)
        else:
            nxt = int(np.argmax(ed))
        want.append(nxt)
        hist.append(nxt)
        lg, _ = om.step(nxt)
    om.close()

    gm = mxhip.Model(p, 128)
    gm.set_logit_edits()
    gm.set_sampling(1, 0.0)
    gm.prefill(prompt[:-1])
    last = int(prompt[-1])
    dev_hist = prompt.tolist()
    for s in range(host_steps):
        lg, _ = gm.step(last)
        ok, err = close_enough(lg, want_host_logits[s])
        assert ok and err < 1e-3, f"host-phase step {s}: logits error {err}"
        order = np.argsort(-edit(lg, dev_hist).astype(np.float64), kind="stable")
        last = int(order[1]) if s == 0 else int(order[0])
        assert last == host_ids[s], f"host-phase step {s}: the host chose {last}, the oracle {host_ids[s]}"
        dev_hist.append(last)
    gm.set_logit_edits(**e)
    if sampled:
        gm.set_sampling(k, temp, seed=seed)
    gm.set_token(last)
    ids, _ = gm.decode(n_dev)
    gm.close()
    assert ids.tolist() == want
    assert not set(e["suppress"]) & set(ids.tolist())


def test_step_errors_are_reported(mxh, tmp_path):
    p = build(tmp_path, "q8-tied")
    gm = mxhip.Model(p, 4)
    with pytest.raises(mxhip.MxhError, match="out of range"):
        gm.step(TINY["n_vocab"])
    with pytest.raises(mxhip.MxhError, match="out of range"):
        gm.set_token(-1)
    # past the 4-row cache the ring keeps going (test_ring_past_full_cache)
    for t in range(6):
        gm.step(t, logits=False)
    # the id history is bounded (2^20 ids): decode and generate refuse a run
    # that would outgrow it before they start
    with pytest.raises(mxhip.MxhError, match="id history"):
        gm.decode(1 << 20)
    with pytest.raises(mxhip.MxhError, match="id history"):
        gm.generate(np.zeros(8, np.int32), 1 << 20)
    with pytest.raises(mxhip.MxhError):
        mxhip.Model(tmp_path / "missing.gguf", 16)


# BASELINE config 1 seeds: (model weights, prompt).  With the first, the
# oracle's smallest top-2 margin over the 64 steps is 8.5e-5 (step 40): a
# near-tie that an error of 1e-4 in the logits would flip.
CONFIG1_SEEDS = [(0x0C0F1, 0xC0F1), (0x1001, 0x2001), (0x1002, 0x2002), (0x1003, 0x2003), (0x1004, 0x2004)]


def oracle_greedy(p, prompt, n, flags, keep_below=0.0):
    """Greedy ids and top-2 margins; the logits of the steps whose margin is
    below keep_below are kept too ({step: logits})."""
    om = mxo.Model(p, 256, flags, threads=16)
    lg = None
    for t in prompt:
        lg, _ = om.step(int(t))
    ids, margins, kept = [], [], {}
    for i in range(n):
        top = np.sort(lg)[-2:]
        margins.append(float(top[1] - top[0]))
        if margins[-1] < keep_below:
            kept[i] = lg.copy()
        nxt = mxo.lib.mxo_argmax(lg.ctypes.data, lg.size)
        ids.append(nxt)
        lg, _ = om.step(nxt)
    om.close()
    return ids, margins, kept


@pytest.mark.parametrize("model_seed,prompt_seed", CONFIG1_SEEDS, ids=[f"{a:x}" for a, _ in CONFIG1_SEEDS])
def test_qwen3_06b_config1_greedy_64_tokens(mxh, tmp_path, model_seed, prompt_seed):
    """Qwen3-0.6B architecture, Q8_0 weights, tied
    embeddings, 32-token seeded prompt (ids uniform in [0, 151936)); the
    first 64 greedy ids, generated free-running (batched prefill, then graph
    decode steps), must be identical to the CPU oracle's, both with the fp16
    KV cache the backend stores and with the reference's fp32 cache."""
    p = tmp_path / "qwen3-0.6b-q8.gguf"
    mxhip.write_synthetic_gguf(p, "qwen3", n_layer=28, n_embd=1024, n_head=16, n_head_kv=8, head_dim=128, n_ff=3072,
                               n_vocab=151936, ctx=40960, qk_norm=True, tied=True, wtype=mxhip.Q8_0,
                               out_type=mxhip.Q8_0, embd_type=mxhip.Q8_0, seed=model_seed, threads=16)
    prompt = np.random.default_rng(prompt_seed).integers(0, 151936, 32).astype(np.int32)
    want16, margins, near = oracle_greedy(p, prompt, 64, mxo.OPEN_KV_FP16, keep_below=1e-3)
    want32, _, _ = oracle_greedy(p, prompt, 64, 0)
    gm = mxhip.Model(p, 256)
    ids, _, _ = gm.generate(prompt, 64)
    gm.close()
    got = ids.tolist()
    for name, want in (("fp16-cache", want16), ("fp32-cache", want32)):
        mism = [i for i in range(64) if got[i] != want[i]]
        assert not mism, (f"{name} oracle: first mismatch at step {mism[0]} (oracle top-2 margin there "
                          f"{margins[mism[0]]:.3g}, smallest margin {min(margins):.3g})")
    # Erosion watch at the near-ties (oracle margin below 1e-3): along the
    # oracle's ids, the device's own gap between the oracle's top two ids and
    # its largest logit difference there.  A gap under half the margin is
    # reported as a warning (seed c0f1, step 40: margin 8.5e-5).
    if near:
        tm = mxhip.Model(p, 256)
        tm.prefill(prompt[:-1])
        lg, _ = tm.step(int(prompt[-1]))
        for i in range(max(near) + 1):
            if i in near:
                olg = near[i]
                b, a = np.argsort(olg)[-2:]
                gap, dmax = float(lg[a] - lg[b]), float(np.abs(lg - olg).max())
                print(f"seed {model_seed:x} step {i}: oracle margin {margins[i]:.3g}, device gap {gap:.3g}, "
                      f"max |dlogit| {dmax:.3g}")
                if gap < 0.5 * margins[i]:
                    warnings.warn(f"config 1 seed {model_seed:x} step {i}: device gap {gap:.3g} under half the "
                                  f"oracle margin {margins[i]:.3g} (max |dlogit| {dmax:.3g})")
            lg, _ = tm.step(want16[i])
        tm.close()
    if model_seed == CONFIG1_SEEDS[0][0]:
        # the prompt token by token through the decode step gives the same ids
        tm = mxhip.Model(p, 256, mxhip.MODEL_TOKEN_PREFILL)
        ids2, _, _ = tm.generate(prompt, 64)
        tm.close()
        assert ids2.tolist() == want16
