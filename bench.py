"""Headline benchmark: Qwen3-8B-shape Q4_K decode at batch 1 on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--prompt P] [--no-cpu-baseline]

Workload: a seeded synthetic GGUF with the
Qwen3-8B architecture (36 layers, hidden 4096, 32/8 heads of 128, FFN 12288,
vocab 151936, QK-norm), every 2D weight Q4_K, the lm-head Q8_0.  A P-token
seeded prompt (default 512) is prefilled (twice: `prefill_tok_s` is the
second call, `prefill_first_call_ms` the first, which also loads the prefill
kernels' code objects), W decode steps warm up, then exactly K greedy decode
steps (default 256) are timed.  A step is one token
through the whole device-resident stack plus the lm-head and argmax.

One JSON line is printed.  `value` is decode tokens/s; `roofline` is for the
dominant kernel, the Q4_K dequant-GEMV, timed with HIP events over every
Q4_K GEMV of the model on its own HBM-resident weights, launched as the
decode step launches them (`traffic` is the HBM bytes per launch that
rocprofv3 counters measured for the same launches, read from the committed
profiles/gemv_q4k_traffic.json, not measured in this run); `cpu_baseline` is
the CPU oracle decoding a bounded sample of the same model on the host
cores.  Also reported: `gemv_microbench` (the isolated
Q4_K GEMV shapes), `long_context` (config 5), and with --all-configs
configs 1 (Qwen3-0.6B) and 4 (Llama-3-8B mixed).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (ROOT / "minxfmr.cpp_amd", ROOT / "oracle"):
    sys.path.insert(0, str(p))

METRIC = "decode tok/s Qwen3-8B-shape Q4_K bs=1; Q4_K GEMV HBM GB/s vs ~8 TB/s peak"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16
ARCH = dict(n_layer=36, n_embd=4096, n_head=32, n_head_kv=8, head_dim=128, n_ff=12288, n_vocab=151936, ctx=40960,
            rope_theta=1e6, eps=1e-6, qk_norm=True, tied=False)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def model_path(seed: int) -> Path:
    d = Path(os.environ.get("MXH_BENCH_DIR", "/tmp"))
    return d / f"mxh_bench_qwen3_8b_q4k_seed{seed}.gguf"


def ensure_model(mxhip, seed: int) -> Path:
    p = model_path(seed)
    if p.exists() and p.stat().st_size > 4_000_000_000:
        return p
    t0 = time.time()
    tmp = p.with_suffix(".tmp")
    mxhip.write_synthetic_gguf(tmp, "qwen3", wtype=mxhip.Q4_K, out_type=mxhip.Q8_0, embd_type=mxhip.Q4_K, seed=seed,
                               threads=min(16, os.cpu_count() or 8), **ARCH)
    tmp.rename(p)
    log(f"wrote synthetic model {p} ({p.stat().st_size / 1e9:.2f} GB) in {time.time() - t0:.1f}s")
    return p


def cpu_model_name() -> str:
    """The host CPU's model name (the `lscpu` 'Model name' field, read from
    /proc/cpuinfo)."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(path: Path, prompt, budget_s: float, threads: int, p0: int, n_ctx: int) -> dict:
    """Oracle decode on the host cores: greedy steps at the positions the
    timed GPU steps run at (from p0 on, the context the bench's prompt and
    warm-up reach) until the time budget is spent, a bounded sample of the
    same workload.  The oracle jumps to p0 instead of prefilling the prompt
    (minutes on the CPU): the cache rows below hold zeros, and the work of a
    step (every weight, and attention over p0 + 1 rows) does not depend on
    their values."""
    import numpy as np

    import mxo

    max_steps = 48
    # the oracle's cache holds its own steps (the GPU run's context may end
    # before p0 + max_steps with few timed steps)
    m = mxo.Model(path, n_ctx=max(n_ctx, p0 + max_steps + 1), threads=threads)
    m.set_pos(p0)
    t0 = time.perf_counter()
    n = 0
    tok = int(prompt[-1])
    while True:
        lg, _ = m.step(tok)
        tok = int(np.argmax(lg))
        n += 1
        el = time.perf_counter() - t0
        if el > budget_s or n >= max_steps:
            break
    m.close()
    return {"value": round(n / el, 4), "unit": "tok/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model_name(),
            "sample": f"{n} greedy decode steps at positions {p0}..{p0 + n - 1} (the timed GPU steps' context; "
                      f"cache rows below zero-filled, same work per step), lm-head included, of the same model by "
                      f"the C oracle with {threads} OpenMP threads, {el:.1f}s"}


def cpu_reference_gemv(budget_s: float, seed: int) -> dict | None:
    """The reference's own CPU GEMV (backend_matmul_rhs_transposed from its
    sources, built into oracle/_ref/libmxref.so with OpenMP) on the four
    Q4_K shapes of BASELINE config 2, random blocks with small finite d, dmin,
    x ~ N(0, 1); each shape repeated within an equal share of the time budget.
    None when the library was not built."""
    import numpy as np

    import mxo

    ref = mxo.load_ref()
    if ref is None:
        return None
    rng = np.random.default_rng(seed + 3)
    shapes, tot_bytes, tot_s = [], 0, 0.0
    for n, k in ((4096, 4096), (12288, 4096), (4096, 12288), (151936, 4096)):
        w = rng.integers(0, 256, n * (k // 256) * 144, dtype=np.uint8).reshape(-1, 144)
        w[:, 0:4] = np.frombuffer(np.array([0x1400, 0x1000], np.uint16).tobytes(), np.uint8)
        x = rng.standard_normal(k, dtype=np.float32)
        y = np.empty(n, np.float32)
        args = (mxo.Q4_K, x.ctypes.data, 1, k, w.ctypes.data, n, y.ctypes.data)
        if ref.ref_matmul_rhs_t(*args) != 0:
            return None
        calls, t0 = 0, time.perf_counter()
        while True:
            ref.ref_matmul_rhs_t(*args)
            calls += 1
            el = time.perf_counter() - t0
            if el > budget_s / 4 or calls >= 200:
                break
        alg = w.nbytes + 4 * k + 4 * n
        shapes.append({"shape": f"{n}x{k}", "us": round(el / calls * 1e6, 1), "gbs": round(alg / (el / calls) / 1e9, 2),
                       "calls": calls})
        tot_bytes += alg
        tot_s += el / calls
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or (os.cpu_count() or 1)
    return {"value": round(tot_bytes / tot_s / 1e9, 2),
            "unit": "GB/s", "cores": threads, "kind": "reference", "cpu_model": cpu_model_name(),
            "sample": "the reference's backend_matmul_rhs_transposed (its CPU sources, OpenMP) on the four Q4_K shapes "
                      "of BASELINE config 2, each repeated for about a quarter of the budget; value = algorithmic bytes "
                      "of one call per shape over the summed per-call times",
            "shapes": shapes}


LLAMA3_MIXED = dict(n_layer=32, n_embd=4096, n_head=32, n_head_kv=8, head_dim=128, n_ff=14336, n_vocab=128256,
                    ctx=8192, rope_theta=5e5, eps=1e-5, qk_norm=False, tied=False)
QWEN3_06B = dict(n_layer=28, n_embd=1024, n_head=16, n_head_kv=8, head_dim=128, n_ff=3072, n_vocab=151936,
                 ctx=40960, rope_theta=1e6, eps=1e-6, qk_norm=True, tied=True)


def extra_model(mxhip, name: str, seed: int) -> Path:
    d = Path(os.environ.get("MXH_BENCH_DIR", "/tmp"))
    p = d / f"mxh_bench_{name}_seed{seed}.gguf"
    if p.exists():
        return p
    tmp = p.with_suffix(".tmp")
    t0 = time.time()
    if name == "llama3_8b_mixed":
        mxhip.write_synthetic_gguf(tmp, "llama", wtype=mxhip.Q4_K, out_type=mxhip.Q8_0, embd_type=mxhip.Q4_K,
                                   attn_v_type=mxhip.Q5_K, ffn_down_type=mxhip.Q5_K, seed=seed,
                                   threads=min(16, os.cpu_count() or 8), **LLAMA3_MIXED)
    else:
        mxhip.write_synthetic_gguf(tmp, "qwen3", wtype=mxhip.Q8_0, out_type=mxhip.Q8_0, embd_type=mxhip.Q8_0,
                                   seed=seed, threads=min(16, os.cpu_count() or 8), **QWEN3_06B)
    tmp.rename(p)
    log(f"wrote {p} ({p.stat().st_size / 1e9:.2f} GB) in {time.time() - t0:.1f}s")
    return p


def run_long_context(mxhip, path: Path, seed: int, flags: int = 0) -> dict:
    """8192-token prompt prefilled in 512-token chunks on
    the matrix cores, then 128 greedy decode tokens against the 8192+ cache.
    `flags` are the model's open flags (MODEL_NO_GRAPH under --eager)."""
    import numpy as np

    n_prompt, n_dec = 8192, 128
    m = mxhip.Model(path, n_prompt + n_dec + 8, flags)
    prompt = np.random.default_rng(seed + 1).integers(0, m.cfg.n_vocab, n_prompt).astype(np.int32)
    _, pf_ms, _ = m.generate(prompt, 1)
    mxhip.synchronize()
    t0 = time.perf_counter()
    m.decode(n_dec)
    mxhip.synchronize()
    dt = time.perf_counter() - t0
    kv_bytes = 2 * m.cfg.n_layer * m.cfg.n_head_kv * m.cfg.head_dim * 2 * (n_prompt + n_dec // 2)
    # the decode attention alone at the final position (every layer, as the
    # step launches it: the grouped kernel and its merge at this context),
    # timed with HIP events on the library stream
    m.bench_attention(1)
    a_ms, a_launch, a_bytes = m.bench_attention(5)
    a_us = a_ms * 1e3 / a_launch
    a_gbs = a_bytes / a_launch / (a_us * 1e-6) / 1e9
    m.close()
    out = {"prompt": n_prompt, "decode_tokens": n_dec, "prefill_tok_s": round(n_prompt / (pf_ms * 1e-3), 1),
           "decode_tok_s": round(n_dec / dt, 2),
           "decode_hbm_gbs": round((m.cfg.step_read_bytes + kv_bytes) / (dt / n_dec) / 1e9, 1),
           "attention_roofline": {"bound": "hbm", "achieved": round(a_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                  "frac": round(a_gbs / HBM_PEAK_GBS, 4), "us_per_layer": round(a_us, 3),
                                  "per_launch_bytes": int(a_bytes / a_launch),
                                  "kernel": "decode attention at L = 8320 (grouped kernel + merge kernel), "
                                            "algorithmic bytes = the K and V rows read"}}
    log(f"long context: {out}")
    return out


def run_gemv_microbench(mxhip, seed: int) -> dict:
    """the isolated Q4_K dequant-GEMV at batch 1 over the
    four listed shapes, with the weights regrouped into the tiled layout
    (mxh_tile_rows) as the model holds them.  Each shape rotates over at least
    512 MB of distinct weight copies (more than the 256 MB Infinity Cache), so
    every launch streams from HBM; 200 launches back to back on the library
    stream, timed with HIP events.  The block bytes are random with small
    finite d, dmin (timing does not depend on the values; parity at these
    shapes is in tests/test_gemv_gpu.py)."""
    import numpy as np

    rng = np.random.default_rng(seed + 2)
    out = []
    for n, k in ((4096, 4096), (12288, 4096), (4096, 12288), (151936, 4096)):
        rb = k // 256 * 144
        wbytes = n * rb
        blocks = rng.integers(0, 256, wbytes, dtype=np.uint8).reshape(-1, 144)
        blocks[:, 0:4] = np.frombuffer(np.array([0x1400, 0x1000], np.uint16).tobytes(), np.uint8)  # d, dmin
        copies = max(2, -(-(512 << 20) // wbytes))
        bufs = []
        for _ in range(copies):
            b = mxhip.DeviceBuffer(wbytes)
            b.upload(blocks)
            tiled = mxhip.tile_rows(mxhip.Q4_K, b, n, k)
            bufs.append(b)
        x = mxhip.DeviceBuffer.from_array(rng.standard_normal(k, dtype=np.float32))
        y = mxhip.DeviceBuffer(4 * n)
        for i in range(10):
            mxhip.gemv(tiled, bufs[i % copies], x, y, n, k)
        mxhip.synchronize()
        launches = 200
        with mxhip.Timer() as tm:
            for i in range(launches):
                mxhip.gemv(tiled, bufs[i % copies], x, y, n, k)
        us = tm.ms * 1e3 / launches
        alg = wbytes + 4 * k + 4 * n
        out.append({"shape": f"{n}x{k}", "algorithmic_bytes": alg, "us": round(us, 2),
                    "gbs": round(alg / us / 1e3, 1), "frac": round(alg / us / 1e3 / HBM_PEAK_GBS, 4),
                    "copies": copies})
        for b in bufs + [x, y]:
            b.close()
    log(f"GEMV microbench: " + ", ".join(f"{r['shape']} {r['us']} us {r['gbs']} GB/s" for r in out))
    return {"type": "Q4_K (tiled layout)", "launches": 200, "shapes": out}


def run_extra_configs(mxhip, seed: int, flags: int = 0) -> dict:
    """BASELINE configs 1 and 4: Qwen3-0.6B Q8_0 greedy (32-token prompt, 128
    tokens) and Llama-3-8B mixed Q4_K/Q5_K with seeded top-k 8, T 0.8 sampling
    (128-token prompt, 512 tokens)."""
    import numpy as np

    res = {}
    for name, n_prompt, n_gen, sampling in (("qwen3_0_6b_q8", 32, 128, None),
                                            ("llama3_8b_mixed", 128, 512, (8, 0.8, 0xC0F3))):
        p = extra_model(mxhip, name, seed)
        m = mxhip.Model(p, n_prompt + n_gen + 8, flags)
        if sampling:
            m.set_sampling(sampling[0], sampling[1], seed=sampling[2])
        prompt = np.random.default_rng(seed + 2).integers(0, m.cfg.n_vocab, n_prompt).astype(np.int32)
        m.generate(prompt, 8)  # warm-up
        ids, pf_ms, dec_ms = m.generate(prompt, n_gen)
        res[name] = {"prompt": n_prompt, "tokens": n_gen, "sampling": "top-k 8, T 0.8, seeded" if sampling else "greedy",
                     "prefill_tok_s": round(n_prompt / (pf_ms * 1e-3), 1),
                     "decode_tok_s": round((n_gen - 1) / (dec_ms * 1e-3), 2),
                     "decode_weight_gbs": round(m.cfg.step_read_bytes / (dec_ms * 1e-3 / (n_gen - 1)) / 1e9, 1)}
        log(f"{name}: {res[name]}")
        m.close()
    return res


def measured_traffic(per_launch_bytes: int):
    """HBM bytes per Q4_K GEMV launch from the committed rocprofv3
    FETCH_SIZE/WRITE_SIZE measurement of the same shapes (None if absent or
    for other shapes)."""
    p = ROOT / "profiles" / "gemv_q4k_traffic.json"
    try:
        d = json.loads(p.read_text())
    except (OSError, ValueError):
        return None
    if int(d.get("per_launch_algorithmic_bytes", -1)) != int(per_launch_bytes):
        return None
    return int(d["traffic_per_launch_bytes"])


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--seed", type=int, default=8)
    ap.add_argument("--gemv-reps", type=int, default=5)
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--eager", action="store_true",
                    help="enqueue kernels directly instead of replaying HIP graphs, in every leg (the mode to profile "
                         "under rocprofv3, whose kernel tracing has ended in a host fault below hipGraphLaunch)")
    ap.add_argument("--no-long-context", action="store_true", help="skip the 8192-token context measurement")
    ap.add_argument("--no-microbench", action="store_true", help="skip the isolated Q4_K GEMV shapes")
    ap.add_argument("--all-configs", action="store_true",
                    help="also run BASELINE configs 1 (Qwen3-0.6B Q8_0) and 4 (Llama-3-8B mixed, sampled)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build targets a single MI355X); --gpus {args.gpus} is not "
              f"supported", file=sys.stderr)
        return 2
    import numpy as np

    import mxhip

    mxhip.init(0)
    path = ensure_model(mxhip, args.seed)
    n_ctx = args.prompt + args.warmup + args.steps + 8
    t0 = time.time()
    model = mxhip.Model(path, n_ctx, mxhip.MODEL_NO_GRAPH if args.eager else 0)
    cfg = model.cfg
    log(f"model in HBM: {cfg.weight_bytes / 1e9:.2f} GB, {time.time() - t0:.1f}s; step reads "
        f"{cfg.step_read_bytes / 1e9:.3f} GB of weights")
    prompt = np.random.default_rng(args.seed).integers(0, cfg.n_vocab, args.prompt).astype(np.int32)

    # prefill + first token, twice: the first call in a process also loads
    # the prefill kernels' code objects (reported as prefill_first_call_ms);
    # the second, from a reset model, is the timed prefill.  Then untimed
    # warmup steps.
    _, prefill_first_ms, _ = model.generate(prompt, 1)
    _, prefill_ms, _ = model.generate(prompt, 1)
    if args.warmup > 0:
        model.decode(args.warmup)
    mxhip.synchronize()
    # timed region: exactly K decode steps, synchronized on both sides
    t_start = time.perf_counter()
    ids, dev_ms = model.decode(args.steps)
    mxhip.synchronize()
    wall_s = time.perf_counter() - t_start
    tok_s = args.steps / wall_s
    log(f"decode: {args.steps} steps in {wall_s * 1e3:.1f} ms wall ({dev_ms:.1f} ms device) -> {tok_s:.1f} tok/s; "
        f"prefill {args.prompt} tokens {prefill_ms:.1f} ms (first call {prefill_first_ms:.1f} ms)")

    # dominant kernel: Q4_K GEMV over the model's own weights
    model.bench_gemv(mxhip.Q4_K, 1)
    g_ms, g_launch, g_bytes = model.bench_gemv(mxhip.Q4_K, args.gemv_reps)
    g_avg_us = g_ms * 1e3 / g_launch
    g_bytes_launch = g_bytes / g_launch
    gemv_gbs = g_bytes_launch / (g_avg_us * 1e-6) / 1e9
    h_ms, h_launch, h_bytes = model.bench_gemv(mxhip.Q8_0, args.gemv_reps)
    log(f"Q4_K GEMV: {g_launch} launches, avg {g_avg_us:.2f} us, {g_bytes_launch / 1e6:.2f} MB/launch -> "
        f"{gemv_gbs:.0f} GB/s; Q8_0 lm-head {h_ms * 1e3 / h_launch:.1f} us -> "
        f"{h_bytes / h_launch / (h_ms * 1e-3 / h_launch) / 1e9:.0f} GB/s")
    step_bytes = cfg.step_read_bytes
    # prefill: every prompt token but the last goes through the batched
    # matrix-core path; linear-layer flops 2 * (weights per token) * tokens
    lin = cfg.n_layer * ((cfg.n_head + 2 * cfg.n_head_kv) * cfg.head_dim * cfg.n_embd
                         + cfg.n_head * cfg.head_dim * cfg.n_embd + 3 * cfg.n_ff * cfg.n_embd)
    pf_flops = 2.0 * lin * (args.prompt - 1)
    model.close()

    out = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_s * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        # the GEMV arithmetic: Q4_K codes times x as 24-bit block fixed point
        # (int8 limb dot products, exact in int32), fp32 scaling and sums
        "dtype": "q4_k x int24 (int32 dot, fp32 accumulate)",
        "data": "synthetic",
        "config": {"workload": f"qwen3-8b-shape, Q4_K weights + Q8_0 lm-head, bs=1: {args.prompt}-token seeded "
                               f"prompt prefill, then {args.steps} timed greedy decode steps",
                   "global_batch": 1, "seq_len": args.prompt + args.warmup + args.steps},
        "decode_weight_gbs": round(step_bytes / (wall_s / args.steps) / 1e9, 1),
        "decode_hbm_frac": round(step_bytes / (wall_s / args.steps) / 1e9 / HBM_PEAK_GBS, 4),
        "prefill_tok_s": round(args.prompt / (prefill_ms * 1e-3), 1),
        "prefill_first_call_ms": round(prefill_first_ms, 2),
        "prefill_roofline": {"bound": "mfma", "achieved": round(pf_flops / (prefill_ms * 1e-3) / 1e12, 1),
                             "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                             "frac": round(pf_flops / (prefill_ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
                             "flops": pf_flops,
                             "kernel": "whole prefill pass; projections on fp16 MFMA (exact Q4_K weight integers, "
                                       "split hi+lo activations)"},
        "roofline": {"bound": "hbm", "achieved": round(gemv_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gemv_gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(g_bytes_launch),
                     "traffic_source": "profiles/gemv_q4k_traffic.json: rocprofv3 FETCH_SIZE + WRITE_SIZE of the "
                                       "same launches, calibrated by a copy of known size (committed, not measured "
                                       "in this run)",
                     "kernel": "Q4_K dequant-GEMV, tiled weight layout (gemv_kernel<Q4KT>), every Q4_K GEMV of "
                               "the decode step as the step launches it (norm-fused q|k|v and gate|up, SwiGLU "
                               "gate|up, residual o and down)",
                     "per_launch_bytes": int(g_bytes_launch), "avg_launch_us": round(g_avg_us, 3)},
    }
    if not args.no_microbench:
        out["gemv_microbench"] = run_gemv_microbench(mxhip, args.seed)
    if not args.no_long_context:
        out["long_context"] = run_long_context(mxhip, path, args.seed, mxhip.MODEL_NO_GRAPH if args.eager else 0)
    if args.all_configs:
        out["configs"] = run_extra_configs(mxhip, args.seed, mxhip.MODEL_NO_GRAPH if args.eager else 0)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(path, prompt, args.cpu_seconds, min(16, os.cpu_count() or 8),
                                           p0=args.prompt + args.warmup, n_ctx=n_ctx)
        if not args.no_microbench:
            ref_gemv = cpu_reference_gemv(8.0, args.seed)
            if ref_gemv:
                out["cpu_baseline_gemv_reference"] = ref_gemv
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
