"""bench.py's CPU baseline leg (CPU).

The leg times the oracle from the position the GPU's timed steps start at,
for up to 48 steps.  With few timed GPU steps (the driver's `--steps 20
--warmup 5`) the GPU run's context ends before that, so the oracle must size
its own cache; this runs the leg on a tiny model in exactly that situation.
"""
from __future__ import annotations

import numpy as np

import bench
import mxhip


def test_cpu_baseline_past_the_gpu_context(tmp_path):
    p = tmp_path / "tiny.gguf"
    mxhip.write_synthetic_gguf(p, "qwen3", seed=3, n_layer=1, n_embd=256, n_head=4, n_head_kv=2, head_dim=64,
                               n_ff=512, n_vocab=100, wtype=mxhip.Q4_K, out_type=mxhip.Q8_0,
                               embd_type=mxhip.Q8_0, qk_norm=True)
    prompt = np.arange(12, dtype=np.int32)
    # the driver's proportions: context p0 + 28, steps from p0 until 48 or the budget
    out = bench.cpu_baseline(p, prompt, budget_s=30.0, threads=2, p0=17, n_ctx=45)
    assert out["value"] > 0 and out["kind"] == "port" and out["cores"] == 2
    assert "positions 17..64" in out["sample"], out["sample"]
    assert out["cpu_model"]
