"""Whole-layer pin of the oracle against the reference's decoder layer.

The oracle's model step (GGUF reader, embedding, layers, cache) is run on a
tiny seeded model and compared per layer with transformer_forward_single_layer
from the reference's own sources: live through oracle/_ref when it is built
here, and always against the trace committed in tests/golden/ref_layer_trace.npz
(produced by tests/golden/make_golden.py from the same seeded model).
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import gguf_synth
import mxo
from layer_trace import RING_SEQ_MAX, RING_TOKENS, TINY, TOKENS, ref_stack_trace

GOLD = Path(__file__).resolve().parent / "golden" / "ref_layer_trace.npz"
GOLD_RING = Path(__file__).resolve().parent / "golden" / "ref_ring_trace.npz"


def oracle_trace(path, tokens=TOKENS, n_ctx=64):
    m = mxo.Model(path, n_ctx=n_ctx, flags=mxo.OPEN_NO_QK_NORM)
    out = []
    for t in tokens:
        _, tr = m.step(t, want_logits=False, trace=True)
        out.append(tr[:-1])
    m.close()
    return np.stack(out)


def test_oracle_layers_vs_committed_reference_trace(tmp_path):
    path = gguf_synth.build(tmp_path / "tiny.gguf", gguf_synth.Arch(**TINY), seed=123)
    gold = np.load(GOLD)
    got = oracle_trace(path)
    want = gold["hidden"]
    assert got.shape == want.shape
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())


@pytest.mark.skipif(mxo.load_ref() is None, reason="reference build (oracle/_ref) not present")
def test_oracle_layers_vs_live_reference(tmp_path):
    keep = {}
    path = gguf_synth.build(tmp_path / "tiny.gguf", gguf_synth.Arch(**TINY), seed=123, keep=keep)
    want = ref_stack_trace(keep, TINY, TOKENS)
    got = oracle_trace(path)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())


def test_oracle_ring_vs_committed_reference_trace(tmp_path):
    """Past a full cache of 5 rows (14 tokens): the oldest row is overwritten
    and RoPE stays at position 5, as in the reference's ring."""
    path = gguf_synth.build(tmp_path / "tiny.gguf", gguf_synth.Arch(**TINY), seed=123)
    gold = np.load(GOLD_RING)
    assert int(gold["seq_max"]) == RING_SEQ_MAX and list(gold["tokens"]) == RING_TOKENS
    got = oracle_trace(path, RING_TOKENS, RING_SEQ_MAX)
    want = gold["hidden"]
    assert got.shape == want.shape
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())
    # the wrap changes the result: a cache as long as the sequence differs
    # after position 5
    unwrapped = oracle_trace(path, RING_TOKENS, 64)
    np.testing.assert_allclose(unwrapped[:RING_SEQ_MAX + 1], want[:RING_SEQ_MAX + 1], rtol=1e-5,
                               atol=1e-5 * np.abs(want).max())
    assert np.abs(unwrapped[RING_SEQ_MAX + 1:] - want[RING_SEQ_MAX + 1:]).max() > 1e-2 * np.abs(want).max()


@pytest.mark.skipif(mxo.load_ref() is None, reason="reference build (oracle/_ref) not present")
def test_oracle_ring_vs_live_reference(tmp_path):
    keep = {}
    path = gguf_synth.build(tmp_path / "tiny.gguf", gguf_synth.Arch(**TINY), seed=123, keep=keep)
    want = ref_stack_trace(keep, TINY, RING_TOKENS, seq_max=RING_SEQ_MAX)
    got = oracle_trace(path, RING_TOKENS, RING_SEQ_MAX)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())
