"""Workloads to run under rocprofv3 and summaries of what it writes.

    # HBM traffic of the model's Q4_K dequant-GEMVs (tiled weight layout) at
    # the Qwen3-8B decode shapes, calibrated against a plain device-to-device
    # copy of known size; MODEL is the bench's synthetic GGUF (bench.py writes
    # it to $MXH_BENCH_DIR, /tmp by default)
    rocprofv3 --pmc FETCH_SIZE -d OUT/fetch -o run --output-format csv -- \
        python3 -m mxhip.profiling workload MODEL
    rocprofv3 --pmc WRITE_SIZE -d OUT/write -o run --output-format csv -- \
        python3 -m mxhip.profiling workload MODEL
    python3 -m mxhip.profiling traffic OUT/fetch OUT/write > summary.md
    # bytes the CUs read from L2 for the same launches
    rocprofv3 --pmc TCP_TCC_READ_REQ_sum -d OUT/l2 -o run --output-format csv -- \
        python3 -m mxhip.profiling workload MODEL
    python3 -m mxhip.profiling l2reads OUT/l2

    # the long-context decode attention (grouped kernel + merge) at L = 8192
    rocprofv3 --pmc FETCH_SIZE -d OUT/lf -o run --output-format csv -- python3 -m mxhip.profiling workload_long MODEL
    rocprofv3 --pmc WRITE_SIZE -d OUT/lw -o run --output-format csv -- python3 -m mxhip.profiling workload_long MODEL
    rocprofv3 --kernel-trace --stats -d OUT/lt -o run --output-format csv -- \
        python3 -m mxhip.profiling workload_long MODEL
    python3 -m mxhip.profiling attn OUT/lf OUT/lw OUT/lt/run_kernel_stats.csv

    # per-kernel time table from a --kernel-trace --stats run
    python3 -m mxhip.profiling stats OUT/trace/run_kernel_stats.csv

    # MFMA utilisation of the prefill kernels: counters in one run, kernel
    # durations from a --kernel-trace --stats run of the same command
    rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE SQ_INSTS_VALU_MFMA_MOPS_F16 \
        SQ_INSTS_VALU_MFMA_MOPS_BF16 -d OUT/mfma -o run --output-format csv -- python3 bench.py --steps 1 \
        --warmup 0 --gemv-reps 1 --no-cpu-baseline --no-long-context
    python3 -m mxhip.profiling mfma OUT/mfma OUT/trace/run_kernel_stats.csv

The workload decodes the bench's context (512-token prompt, position 528:
the o-projection merges four attention splits), then runs every Q4_K GEMV
of the model (per layer: fused q|k|v, o, fused gate|up, down) `reps` times,
as the bench's roofline pass does, and copies 256 MiB once per rep.  FETCH_SIZE and WRITE_SIZE are reported by
rocprofv3 in KiB per dispatch; the calibration factor is the copy's known
byte count divided by what the counter reads for it.
"""
from __future__ import annotations

import csv
import glob
import os
import re
import sys
from pathlib import Path

# Q4_K GEMV shapes of one Qwen3-8B layer (out x in): fused q|k|v, o,
# fused gate|up, down
SHAPES = [("qkv", 6144, 4096), ("o", 4096, 4096), ("gate_up", 24576, 4096), ("down", 4096, 12288)]
N_LAYER = 36
COPY_BYTES = 256 << 20


def algorithmic_bytes(n: int, k: int) -> int:
    """Q4_K GEMV: N*K/256*144 weight bytes + 4K (x) + 4N (y)."""
    return n * k // 256 * 144 + 4 * k + 4 * n


# the bench's context: a 512-token prompt, 16 warm-up steps and 256 timed
# ones fit 792 positions (four attention splits in the grid); the workload
# decodes to position 528, so the o-projection merges four live splits
BENCH_CTX, BENCH_PROMPT, BENCH_STEPS = 792, 512, 17


def workload(path: str, reps: int = 4) -> None:
    import numpy as np

    import mxhip

    mxhip.init(0)
    m = mxhip.Model(path, BENCH_CTX, mxhip.MODEL_NO_GRAPH)  # profiled runs stay off graph replay
    prompt = np.random.default_rng(8).integers(0, m.cfg.n_vocab, BENCH_PROMPT).astype(np.int32)
    m.generate(prompt, BENCH_STEPS)
    src = mxhip.DeviceBuffer(COPY_BYTES)
    dst = mxhip.DeviceBuffer(COPY_BYTES)
    mxhip.memset(src, 1)
    for _ in range(reps):
        m.bench_gemv(mxhip.Q4_K, 1)
        mxhip.copy(dst, src, COPY_BYTES)
        m.bench_gemv(mxhip.Q8_0, 1)  # the 661 MB lm-head: a second stream of known size
    mxhip.synchronize()
    m.close()
    print(f"[workload] {reps} passes over the model's Q4_K GEMVs, copy {COPY_BYTES} B each", file=sys.stderr,
          flush=True)


# the long-context workload: an 8192-token prompt, then
# decode steps at L = 8192 .. with the grouped attention kernel
LONG_PROMPT, LONG_STEPS = 8192, 8


def workload_long(path: str) -> None:
    import numpy as np

    import mxhip

    mxhip.init(0)
    m = mxhip.Model(path, LONG_PROMPT + LONG_STEPS + 8, mxhip.MODEL_NO_GRAPH)  # profiled runs stay off graph replay
    prompt = np.random.default_rng(55).integers(0, m.cfg.n_vocab, LONG_PROMPT).astype(np.int32)
    # the prompt in 1024-token pieces (batched prefill, 512-token chunks),
    # reporting each: under --pmc every dispatch is serialized
    for i in range(0, LONG_PROMPT - 1, 1024):
        m.prefill(prompt[i:min(i + 1024, LONG_PROMPT - 1)])
        mxhip.synchronize()
        print(f"[workload_long] prefilled {min(i + 1024, LONG_PROMPT - 1)} tokens", file=sys.stderr, flush=True)
    lg, _ = m.step(int(prompt[-1]))
    m.set_token(int(np.argmax(lg)))
    m.decode(LONG_STEPS - 1)
    mxhip.synchronize()
    print(f"[workload_long] decoded {LONG_STEPS} steps", file=sys.stderr, flush=True)
    src = mxhip.DeviceBuffer(COPY_BYTES)
    dst = mxhip.DeviceBuffer(COPY_BYTES)
    mxhip.memset(src, 1)
    mxhip.copy(dst, src, COPY_BYTES)
    mxhip.synchronize()
    m.close()
    print(f"[workload_long] {LONG_PROMPT}-token prompt, {LONG_STEPS} decode steps, copy {COPY_BYTES} B",
          file=sys.stderr, flush=True)


def attn(fetch_dir: str, write_dir: str, stats_csv: str | None = None) -> None:
    """HBM bytes per decode-attention dispatch of workload_long (the grouped
    kernel and its merge kernel), calibrated by the copy as in `traffic`,
    against the K/V rows the step reads: 2 L n_kv hd 2 bytes at L = pos + 1
    (Qwen3-8B: n_kv 8, hd 128; 36 dispatches per step)."""
    rows_f, rows_w = _counter_rows(fetch_dir), _counter_rows(write_dir)

    def ordered(rows, counter, pick):
        acc: dict[int, float] = {}
        for r in rows:
            if r.get("Counter_Name") == counter and pick(r["Kernel_Name"]):
                acc[int(r["Dispatch_Id"])] = acc.get(int(r["Dispatch_Id"]), 0.0) + float(r["Counter_Value"])
        return sorted(acc.items())

    grp = lambda n: "attention_group_kernel" in n
    mrg = lambda n: "attention_merge_kernel" in n
    cpy = lambda n: "copy" in n.lower()
    af, aw = ordered(rows_f, "FETCH_SIZE", grp), ordered(rows_w, "WRITE_SIZE", grp)
    mf, mw = ordered(rows_f, "FETCH_SIZE", mrg), ordered(rows_w, "WRITE_SIZE", mrg)
    if not af or not aw:
        raise SystemExit("no attention_group_kernel dispatch found")
    cf = _big([v for k, v in ordered(rows_f, "FETCH_SIZE", cpy) if k > af[0][0]])
    cw = _big([v for k, v in ordered(rows_w, "WRITE_SIZE", cpy) if k > aw[0][0]])
    if not cf or not cw:
        raise SystemExit("no calibration copy found")
    kib = COPY_BYTES / 1024
    f_cal, w_cal = kib / (sum(cf) / len(cf)), kib / (sum(cw) / len(cw))
    n_kv, hd = 8, 128
    steps = len(af) // N_LAYER
    # the first step (the prompt's last token) is at pos LONG_PROMPT - 1
    alg = [2 * (LONG_PROMPT + i) * n_kv * hd * 2 for i in range(steps)]
    fb = [v * 1024 * f_cal for _, v in af]
    wb = [v * 1024 * w_cal for _, v in aw]
    a_avg = sum(alg[i // N_LAYER] for i in range(len(fb))) / len(fb)
    print("| dispatch | K/V bytes read (algorithmic) | FETCH (scaled) B | WRITE (scaled) B | traffic / algorithmic |")
    print("|---|---:|---:|---:|---:|")
    print(f"| `attention_group_kernel<16, 4>`, {len(fb)} dispatches ({steps} steps x {N_LAYER} layers) | "
          f"{a_avg:,.0f} | {sum(fb) / len(fb):,.0f} | {sum(wb) / len(wb):,.0f} | "
          f"{(sum(fb) + sum(wb)) / len(fb) / a_avg:.3f} |")
    if mf and mw:
        print(f"| `attention_merge_kernel`, {len(mf)} dispatches | - | {sum(v for _, v in mf) / len(mf) * 1024 * f_cal:,.0f} "
              f"| {sum(v for _, v in mw) / len(mw) * 1024 * w_cal:,.0f} | - |")
    print()
    print(f"Calibration: factors {f_cal:.4f} (fetch) and {w_cal:.4f} (write) from a {COPY_BYTES:,} B copy.")
    if stats_csv:
        with open(stats_csv, newline="") as fh:
            for r in csv.DictReader(fh):
                if "attention_group_kernel" in r["Name"] or "attention_merge_kernel" in r["Name"]:
                    us = float(r["AverageNs"]) / 1e3
                    extra = ""
                    if "attention_group_kernel" in r["Name"]:
                        extra = f", {a_avg / (us * 1e-6) / 1e9:,.0f} GB/s of K/V, {a_avg / (us * 1e-6) / 8e12:.3f} of 8 TB/s"
                    name = re.sub(r"\([^()]*\)$", "", r["Name"].replace("mxh::(anonymous namespace)::", "").replace("mxh::", "").replace("void ", ""))
                    print(f"`{name}`: {r['Calls']} dispatches, average {us:.2f} us{extra}")


def _counter_rows(d: str):
    files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no counter_collection.csv under {d}")
    rows = []
    for f in files:
        with open(f, newline="") as fh:
            rows.extend(csv.DictReader(fh))
    return rows


def _per_dispatch(rows, counter: str, reduce=None):
    """{kernel name: [value per dispatch]} for one counter, combining the
    per-instance rows rocprofv3 may write for a dispatch with `reduce`
    (sum by default; max for whole-device clocks such as GRBM_GUI_ACTIVE)."""
    reduce = reduce or (lambda a, b: a + b)
    acc: dict[tuple[str, str], float] = {}
    for r in rows:
        if r.get("Counter_Name") != counter:
            continue
        key = (r["Dispatch_Id"], r["Kernel_Name"])
        v = float(r["Counter_Value"])
        acc[key] = reduce(acc[key], v) if key in acc else v
    out: dict[str, list[float]] = {}
    for (did, name), v in sorted(acc.items(), key=lambda kv: int(kv[0][0])):
        out.setdefault(name, []).append(v)
    return out


def _big(vals):
    """The calibration copies among copy dispatches: those of the largest
    size (the runtime's own small copies, such as the id read-back of a
    decode, are left out)."""
    top = max(vals, default=0.0)
    return [v for v in vals if v > 0.9 * top]


def traffic(fetch_dir: str, write_dir: str) -> None:
    rows_f = _counter_rows(fetch_dir)
    rows_w = _counter_rows(write_dir)

    def ordered(rows, counter, pick):
        acc: dict[int, float] = {}
        for r in rows:
            if r.get("Counter_Name") == counter and pick(r["Kernel_Name"]):
                acc[int(r["Dispatch_Id"])] = acc.get(int(r["Dispatch_Id"]), 0.0) + float(r["Counter_Value"])
        return sorted(acc.items())

    def is_gemv(n):
        return "gemv_kernel" in n and "Q4KT" in n

    def is_copy(n):
        return "copy" in n.lower()

    # Q4_K GEMV dispatches in issue order (both epilogues): per layer q|k|v,
    # o, gate|up, down; the first pass is skipped (cold instruction and TLB
    # state).  The calibration copies are the copy dispatches after the first
    # GEMV (model loading also issues small copies).
    gf, gw = ordered(rows_f, "FETCH_SIZE", is_gemv), ordered(rows_w, "WRITE_SIZE", is_gemv)
    if not gf or not gw:
        raise SystemExit("no Q4_K GEMV dispatch found")
    cf = _big([v for k, v in ordered(rows_f, "FETCH_SIZE", is_copy) if k > gf[0][0]])
    cw = _big([v for k, v in ordered(rows_w, "WRITE_SIZE", is_copy) if k > gw[0][0]])
    if not cf or not cw:
        raise SystemExit("no calibration copy found")
    kib = COPY_BYTES / 1024
    copy_f, copy_w = sum(cf) / len(cf), sum(cw) / len(cw)
    f_cal, w_cal = kib / copy_f, kib / copy_w
    fv, wv = [v for _, v in gf], [v for _, v in gw]
    per_pass = 4 * N_LAYER
    if len(fv) < 2 * per_pass or len(fv) % per_pass or len(wv) != len(fv):
        raise SystemExit(f"unexpected Q4_K GEMV dispatch count {len(fv)} / {len(wv)}")
    print("| shape (N x K) | algorithmic B | FETCH (scaled) B | WRITE (scaled) B | traffic / algorithmic |")
    print("|---|---:|---:|---:|---:|")
    tot_alg = tot_traffic = 0.0
    for i, (name, n, k) in enumerate(SHAPES):
        fs = [fv[j] for j in range(per_pass, len(fv)) if j % 4 == i]
        ws = [wv[j] for j in range(per_pass, len(wv)) if j % 4 == i]
        fb = sum(fs) / len(fs) * 1024 * f_cal
        wb = sum(ws) / len(ws) * 1024 * w_cal
        alg = algorithmic_bytes(n, k)
        tot_alg += alg
        tot_traffic += fb + wb
        print(f"| {name} {n} x {k} | {alg:,} | {fb:,.0f} | {wb:,.0f} | {(fb + wb) / alg:.3f} |")
    print(f"| mean per launch | {tot_alg / len(SHAPES):,.0f} | | | {tot_traffic / tot_alg:.3f} |")
    print()
    print(f"Calibration: a {COPY_BYTES:,} B device-to-device copy reads FETCH_SIZE "
          f"{copy_f:,.0f} KiB and WRITE_SIZE {copy_w:,.0f} KiB per dispatch; factors "
          f"{f_cal:.4f} (fetch) and {w_cal:.4f} (write) are applied above.")
    print(f"TRAFFIC_PER_LAUNCH_BYTES={tot_traffic / len(SHAPES):.0f}")


def l2reads(d: str, counter: str = "TCP_TCC_READ_REQ_sum") -> None:
    """Bytes the vector L1 caches (TCP) request from the L2 (TCC) per Q4_K
    GEMV launch of the workload, calibrated by the copy (its known read bytes
    over the requests it issues), against the launch's algorithmic bytes:
    above 1, the CUs read the same lines from L2 more than once (the
    o-projection's staging reads every attention split's partials in every
    workgroup)."""
    rows = _counter_rows(d)
    acc: dict[int, tuple[str, float]] = {}
    for r in rows:
        if r.get("Counter_Name") == counter:
            i = int(r["Dispatch_Id"])
            name, v = acc.get(i, (r["Kernel_Name"], 0.0))
            acc[i] = (name, v + float(r["Counter_Value"]))
    items = sorted(acc.items())
    gemv = [(i, v) for i, (n, v) in items if "gemv_kernel" in n and "Q4KT" in n]
    copies = _big([v for i, (n, v) in items if "copy" in n.lower() and gemv and i > gemv[0][0]])
    if not gemv or not copies:
        raise SystemExit("no Q4_K GEMV or calibration copy dispatch found")
    per_req = COPY_BYTES / (sum(copies) / len(copies))
    vals = [v for _, v in gemv]
    per_pass = 4 * N_LAYER
    print(f"| shape (N x K) | algorithmic B | L2-to-CU read (scaled) B | L2 reads / algorithmic |")
    print("|---|---:|---:|---:|")
    for j, (name, n, k) in enumerate(SHAPES):
        vs = [vals[i] for i in range(per_pass, len(vals)) if i % 4 == j]
        b = sum(vs) / len(vs) * per_req
        alg = algorithmic_bytes(n, k)
        print(f"| {name} {n} x {k} | {alg:,} | {b:,.0f} | {b / alg:.3f} |")
    print()
    print(f"Calibration: the {COPY_BYTES:,} B copy issues {sum(copies) / len(copies):,.0f} {counter} "
          f"requests per dispatch, {per_req:.1f} B each.")


def rdreq(d: str) -> None:
    """Bytes the L2 reads from memory per dispatch from the request counts by
    size (TCC_EA0_RDREQ_32B / _64B / _128B, summed over instances), next to
    the algorithmic bytes: for the Q4_K GEMVs per shape, the copy, and the
    Q8_0 lm-head (661 MB streamed once per pass)."""
    rows = _counter_rows(d)
    per: dict[int, dict] = {}
    for r in rows:
        e = per.setdefault(int(r["Dispatch_Id"]), {"name": r["Kernel_Name"]})
        e[r["Counter_Name"]] = e.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])

    def nbytes(e):
        return 32 * e.get("TCC_EA0_RDREQ_32B_sum", 0) + 64 * e.get("TCC_EA0_RDREQ_64B_sum", 0) + \
            128 * e.get("TCC_EA0_RDREQ_128B_sum", 0)

    items = sorted(per.items())
    gemv = [e for _, e in items if "gemv_kernel" in e["name"] and "Q4KT" in e["name"]]
    first = next(i for i, e in items if "gemv_kernel" in e["name"] and "Q4KT" in e["name"])
    copies = [e for i, e in items if "copy" in e["name"].lower() and i > first]
    big = max((nbytes(e) for e in copies), default=0.0)
    copies = [e for e in copies if nbytes(e) > 0.9 * big]
    heads = [e for i, e in items if "gemv_kernel" in e["name"] and "Q80T" in e["name"] and i > first]
    per_pass = 4 * N_LAYER
    print("| dispatch | algorithmic B | read B (32 / 64 / 128-byte requests) | read / algorithmic | "
          "requests 32 / 64 / 128 B (share) |")
    print("|---|---:|---:|---:|---|")

    def row(label, es, alg):
        b = sum(nbytes(e) for e in es) / len(es)
        n = [sum(e.get(f"TCC_EA0_RDREQ_{w}B_sum", 0) for e in es) for w in (32, 64, 128)]
        tot = sum(n) or 1
        print(f"| {label} | {alg:,} | {b:,.0f} | {b / alg:.3f} | "
              f"{' / '.join(f'{100 * x / tot:.0f}%' for x in n)} |")

    for j, (name, n, k) in enumerate(SHAPES):
        row(f"Q4_K {name} {n} x {k}", [gemv[i] for i in range(per_pass, len(gemv)) if i % 4 == j],
            algorithmic_bytes(n, k))
    if copies:
        row("copy (device to device)", copies, COPY_BYTES)
    if heads:
        row("Q8_0 lm-head 151936 x 4096", heads, 151936 * 4096 // 32 * 34 + 4 * 4096 + 4 * 151936)


def mfma(d: str, stats_csv: str | None = None) -> None:
    """Per-kernel MFMA utilisation from a run with
    --pmc SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE SQ_INSTS_VALU_MFMA_MOPS_F16 SQ_INSTS_VALU_MFMA_MOPS_BF16:
    busy cycles / (GUI-active cycles x SIMDs) (rocprofv3's MfmaUtil), and the
    fp16 + bf16 MFMA flops issued (512 per MOP).  With the kernel stats CSV of
    a --kernel-trace --stats run of the same command, also the issued flop
    rate over each kernel's average duration, against the 2.5 PFLOP/s dense
    fp16/bf16 peak."""
    rows = _counter_rows(d)
    simds = None
    agent = glob.glob(os.path.join(d, "**", "*agent_info.csv"), recursive=True)
    if agent:
        with open(agent[0], newline="") as fh:
            for r in csv.DictReader(fh):
                if r.get("Agent_Type", "").upper() == "GPU" or r.get("Type", "").upper() == "GPU":
                    simds = int(r.get("Simd_Count") or r.get("SIMD_Count") or 0) or None
    busy = _per_dispatch(rows, "SQ_VALU_MFMA_BUSY_CYCLES")
    gui = _per_dispatch(rows, "GRBM_GUI_ACTIVE", max)
    mops = {}
    for cnt in ("SQ_INSTS_VALU_MFMA_MOPS_F16", "SQ_INSTS_VALU_MFMA_MOPS_BF16"):
        for name, vals in _per_dispatch(rows, cnt).items():
            acc = mops.setdefault(name, [0.0] * len(vals))
            for i, v in enumerate(vals):
                acc[i] += v
    dur_us = {}
    if stats_csv:
        with open(stats_csv, newline="") as fh:
            for r in csv.DictReader(fh):
                dur_us[r["Name"]] = float(r["AverageNs"]) / 1e3
    simds = simds or 1024
    short = lambda name: re.sub(r"\([^()]*\)$", "", name.replace("mxh::(anonymous namespace)::", "").replace("void ", ""))
    print("| kernel | dispatches | MFMA busy (% of SIMD cycles) | MFMA GFLOP issued per dispatch | avg us "
          "| issued TFLOP/s | % of 2.5 PFLOP/s |")
    print("|---|---:|---:|---:|---:|---:|---:|")
    for name in busy:
        if name not in gui:
            continue
        b, g = busy[name], gui[name]
        util = 100.0 * sum(b) / (sum(g) * simds) if sum(g) else 0.0
        m = mops.get(name, [0.0])
        fl = sum(m) * 512 / max(1, len(m)) / 1e9
        us = next((v for k, v in dur_us.items() if short(k) == short(name)), None)
        if us:
            tflops = fl / us * 1e3  # GFLOP per us = PFLOP/s
            print(f"| `{short(name)}` | {len(b)} | {util:.1f} | {fl:.1f} | {us:.1f} | {tflops:.0f} | "
                  f"{100.0 * tflops / 2500.0:.1f} |")
        else:
            print(f"| `{short(name)}` | {len(b)} | {util:.1f} | {fl:.1f} | - | - | - |")
    print(f"\nSIMDs: {simds}")


def stats(path: str, top: int = 15) -> None:
    with open(path, newline="") as fh:
        rows = list(csv.DictReader(fh))
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    tot = sum(float(r["TotalDurationNs"]) for r in rows)
    print("| kernel | calls | avg us | total ms | share |")
    print("|---|---:|---:|---:|---:|")
    for r in rows[:top]:
        name = r["Name"].replace("mxh::(anonymous namespace)::", "").replace("mxh::", "").replace("void ", "")
        name = re.sub(r"\([^()]*\)$", "", name)  # argument list
        print(f"| `{name}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
              f"{float(r['TotalDurationNs']) / 1e6:.2f} | {100 * float(r['TotalDurationNs']) / tot:.1f}% |")
    q = [r for r in rows if "gemv_kernel" in r["Name"] and "Q4K" in r["Name"]]
    if q:
        calls = sum(int(r["Calls"]) for r in q)
        print()
        print(f"All Q4_K GEMV dispatches (every epilogue): {calls} calls, average "
              f"{sum(float(r['TotalDurationNs']) for r in q) / calls / 1e3:.2f} us")


def main(argv: list[str]) -> int:
    if not argv:
        print(__doc__)
        return 2
    cmd = argv[0]
    if cmd == "workload":
        workload(argv[1], int(argv[2]) if len(argv) > 2 else 4)
    elif cmd == "workload_long":
        workload_long(argv[1])
    elif cmd == "attn":
        attn(argv[1], argv[2], argv[3] if len(argv) > 3 else None)
    elif cmd == "traffic":
        traffic(argv[1], argv[2])
    elif cmd == "rdreq":
        rdreq(argv[1])
    elif cmd == "l2reads":
        l2reads(argv[1], *argv[2:3])
    elif cmd == "stats":
        stats(argv[1])
    elif cmd == "mfma":
        mfma(argv[1], argv[2] if len(argv) > 2 else None)
    else:
        print(__doc__)
        return 2
    return 0


if __name__ == "__main__":
    sys.path.insert(0, str(Path(__file__).resolve().parent.parent))
    sys.exit(main(sys.argv[1:]))
