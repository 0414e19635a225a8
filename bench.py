"""bench.py — training throughput of the BASELINE model on one MI355X.

Workload (the metric's configuration): one full
training step = forward + backward + AdamW of the d512/8h/4L/seq512 model at
bs 32 (16384 tokens) through the HIP kernels (GEMM, FlashAttention, fused CE,
AdamW), on synthetic uniform tokens and random-init weights.

  python bench.py [--gpus 1] [--steps 20] [--warmup 5]

Prints ONE JSON line. ``value`` = tokens/s over the timed steps (inputs and
weights already resident in HBM). ``roofline`` = the dominant kernel's
algorithmic work per launch / its mean duration, timed with HIP events on the
stream it is launched on during the timed steps. ``cpu_baseline`` = the NumPy
restatement of the same step (the oracle) on the host's cores, bs 4 sample.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from collections import defaultdict

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E


def _args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--batch-size", type=int, default=32)
    ap.add_argument("--seq-len", type=int, default=512)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-variant", action="store_true",
                    help="skip configs[4]'s bs4 x seq4096 variant (timed after the headline workload)")
    ap.add_argument("--no-graph", action="store_true", help="launch every kernel from Python (no HIP graph)")
    ap.add_argument("--torch-step", action="store_true",
                    help="time the same training step written with plain PyTorch ops (a reference point)")
    ap.add_argument("--kernel-configs", action="store_true",
                    help="time BASELINE configs[1] (flash) and configs[3] (CE) in isolation, beside torch's kernels")
    ap.add_argument("--gemm-compare", action="store_true",
                    help="time the BASELINE GEMM products here and through torch.matmul (hipBLASLt)")
    ap.add_argument("--fused-lmhead", action="store_true",
                    help="the loss through linear_cross_entropy (no logits kept between forward and backward)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="run only the LM-head GEMM and a 1 GiB copy (for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--cpu-seconds", type=float, default=20.0, help="budget of the CPU baseline sample")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="write profiles/traffic.json from the rocprofv3 CSV output of the two --pmc runs "
                         "(FETCH_SIZE, WRITE_SIZE) over --traffic-probe")
    ap.add_argument("--replay-probe", action="store_true",
                    help="only warm up, capture and replay the graphed step --steps times (for rocprofv3 "
                         "--kernel-trace: the busy ratio of graph replays)")
    ap.add_argument("--trace-summary", nargs="+", metavar="ARG",
                    help="TRACE_DIR OUT.md TITLE COMMAND STEPS [BENCH_JSON KERNEL]: per-kernel table of a "
                         "rocprofv3 --kernel-trace csv run, for profiles/")
    ap.add_argument("--busy-summary", metavar="TRACE_DIR",
                    help="write profiles/busy_<workload>.json from the rocprofv3 kernel trace of --replay-probe")
    ap.add_argument("--flash-probe", nargs=2, type=int, metavar=("N_HEADS", "SEQ"),
                    help="only run flash forward + backward at (N_HEADS, SEQ, 64) a few times (for rocprofv3 --pmc)")
    ap.add_argument("--pmc-summary", nargs="+", metavar="ARG",
                    help="OUT.md TITLE DIR [DIR ...]: per-kernel PMC medians from rocprofv3 --pmc CSV dirs, with "
                         "MFMA busy, VALU/MFMA and LDS bank-conflict ratios")
    return ap.parse_args()


class KernelProbe:
    """Brackets every libnlearn_hip call with HIP events on the current stream
    (the stream the kernel is launched on)."""

    def __init__(self, torch):
        self.torch = torch
        self.pending = []
        self.enabled = False

    @staticmethod
    def tag(name, args):
        if name in ("nl_gemm", "nl_gemm_ex", "nl_gemm_fused"):
            opA, opB, M, N, K = args[1:6]
            e = args[16] if name == "nl_gemm_fused" else 0
            epi = ("", "_bias", "_bias_gelu", "_dgelu")[e]
            # algorithmic bytes: bf16 operands, C at its dtype (read back too when
            # beta != 0), the saved GELU input written (bias_gelu) or read (dgelu)
            c_bytes = 4 if args[13] == 0 else 2
            byt = 2.0 * (M * K + K * N) + M * N * c_bytes * (2 if args[11] != 0.0 else 1)
            if e in (2, 3):
                byt += 2.0 * M * N
            return f"gemm_{'NT'[opA]}{'NT'[opB]}_{M}x{N}x{K}{epi}", 2.0 * M * N * K, "flops", byt
        if name == "nl_ce_fwd_bwd":
            M, V = args[1:3]
            return f"ce_fwd_bwd_{M}x{V}", 4.0 * M * V + 12.0 * M, "bytes"
        if name == "nl_lce_fwd":
            M, D, V = args[1:4]
            return f"lce_fwd_{M}x{V}x{D}", 2.0 * M * V * D, "flops"
        if name == "nl_lce_bwd_dlogits":
            M, D, V, _, vn = args[1:6]
            return f"lce_dlogits_{M}x{vn}x{D}", 2.0 * M * vn * D, "flops"
        if name == "nl_flash_attention_fwd":
            B, H, S, D = args[1:5]
            f = 2.0 * B * H * S * S * D if args[6] else 4.0 * B * H * S * S * D
            return f"flash_fwd_{B * H}x{S}x{D}", f, "flops"
        if name == "nl_flash_attention_bwd":
            B, H, S, D = args[1:5]
            f = 2.0 * B * H * S * S * D if args[6] else 4.0 * B * H * S * S * D
            return f"flash_bwd_{B * H}x{S}x{D}", 2.5 * f, "flops"
        # the training step launches the backward's kernels one by one (dQ on a
        # second stream): executed products per kernel, S = QK^T and dP = dO V^T
        # counted in both (dK/dV: S, dP, dV, dK; dQ: S, dP, dQ)
        if name in ("nl_flash_attention_bwd_dkdv", "nl_flash_attention_bwd_dq"):
            B, H, S, D = args[1:5]
            f = 2.0 * B * H * S * S * D if args[6] else 4.0 * B * H * S * S * D
            which = "dkdv" if name.endswith("dkdv") else "dq"
            return f"flash_bwd_{which}_{B * H}x{S}x{D}", (2.0 if which == "dkdv" else 1.5) * f, "flops"
        if name == "nl_flash_attention_bwd_preprocess":
            B, H, S, D = args[1:5]
            return f"flash_bwd_pre_{B * H}x{S}x{D}", 2.0 * 2 * B * H * S * D + 4.0 * B * H * S, "bytes"
        return None

    def __call__(self, name, args):
        if not self.enabled:
            return None
        t = self.tag(name, args)
        if t is None:
            return None
        probe = self

        class _Ctx:
            def __enter__(self_inner):
                self_inner.e0 = probe.torch.cuda.Event(enable_timing=True)
                self_inner.e1 = probe.torch.cuda.Event(enable_timing=True)
                self_inner.e0.record()

            def __exit__(self_inner, *exc):
                self_inner.e1.record()
                probe.pending.append((t, self_inner.e0, self_inner.e1))
                return False

        return _Ctx()

    def summary(self, steps):
        agg = defaultdict(lambda: [0.0, 0, 0.0, "", None])
        for (tag, work, kind, *byt), e0, e1 in self.pending:
            a = agg[tag]
            a[0] += e0.elapsed_time(e1) * 1e-3
            a[1] += 1
            a[2] = work
            a[3] = kind
            a[4] = byt[0] if byt else None
        out = {}
        for tag, (tot, n, work, kind, byt) in agg.items():
            avg = tot / n
            rate = work / avg
            if kind == "flops":
                # the attainable roof: min(MFMA peak, arithmetic intensity x HBM
                # bandwidth) when the algorithmic bytes are known (GEMMs)
                peak, bound = PEAK_BF16_TFLOPS, "mfma"
                if byt:
                    hbm_roof = work / byt * PEAK_HBM_GBS / 1e3
                    if hbm_roof < peak:
                        peak, bound = hbm_roof, "hbm"
                out[tag] = {"bound": bound, "achieved": rate / 1e12, "peak": round(peak, 1),
                            "unit": "TFLOP/s", "avg_us": avg * 1e6, "launches_per_step": n / steps,
                            "time_per_step_ms": tot / steps * 1e3, "work_per_launch": work}
                if byt:
                    out[tag]["bytes_per_launch"] = byt
                    out[tag]["intensity"] = round(work / byt, 1)
            else:
                out[tag] = {"bound": "hbm", "achieved": rate / 1e9, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                            "avg_us": avg * 1e6, "launches_per_step": n / steps,
                            "time_per_step_ms": tot / steps * 1e3, "work_per_launch": work}
            out[tag]["frac"] = out[tag]["achieved"] / out[tag]["peak"]
        return out


def cpu_baseline(seconds: float):
    """Time the NumPy restatement of the training step (bs 4, seq 512) on the host."""
    import numpy as np

    from oracle import model_np

    cores = len(os.sched_getaffinity(0))
    bs, seq = 4, 512
    step = model_np.TrainStepNP(model_np.init_params(0), lr=3e-4)
    rng = np.random.default_rng(0)
    batch = rng.integers(0, 50257, (bs, seq + 1)).astype(np.int64)
    t0 = time.time()
    for _ in range(2):  # warm-up (page-in, BLAS threads), as the CPU-baseline plan asks
        step(batch)
    times = []
    while True:
        t1 = time.time()
        step(batch)
        times.append(time.time() - t1)
        if time.time() - t0 > seconds or len(times) >= 5:
            break
    t = float(np.median(times))
    return {"value": bs * seq / t, "unit": "tokens/s", "cores": cores, "kind": "port",
            "cpu_model": _cpu_model(),
            "sample": f"NumPy fp32 restatement of one train step (fwd+bwd+AdamW), bs {bs} x seq {seq}, "
                      f"median of {len(times)} steps after 2 warm-ups; {t:.2f} s/step"}


def _cpu_model() -> str:
    """The host CPU's model name (what lscpu prints as 'Model name')."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")


# The products --traffic-probe runs, in launch order within one repetition:
# (tag, M, N, K, algorithmic bytes). The LM head's three GEMMs, then the four
# layer weight-gradient products X^T dY at M = 16384 tokens (fp32 outputs, K
# split into fp32 partials that a second kernel reduces).
def _traffic_products():
    T, d, f, V = 16384, 512, 2048, 50257
    from nlearn_amd.kernels.cross_entropy import chunk_bounds

    h = chunk_bounds(T, 2)[1]   # the training step's logits GEMM runs in two row chunks; the first
    prods = [("gemm_NN_16384x50257x512", 2 * (T * d + d * V + T * V)),
             ("gemm_NT_16384x512x50257", 2 * (T * V + d * V + T * d)),
             ("gemm_TN_512x50257x16384", 2 * (T * d + T * V) + 4 * d * V),
             (f"gemm_NN_{h}x50257x512", 2 * (h * d + d * V + h * V))]
    for kin, nout in ((d, 3 * d), (d, d), (d, f), (f, d)):
        prods.append((f"gemm_TN_{kin}x{nout}x{T}", 2 * (T * kin + T * nout) + 4 * kin * nout))
    return prods


def traffic_probe(reps: int = 5) -> None:
    """The LM-head GEMMs (forward NN, input-gradient NT with its K split and
    reduction, weight-gradient TN) and the layer weight-gradient TN products
    alone at the bench shapes, on inputs with the training step's statistics,
    each repetition ending with a plain 1 GiB device copy: the known-size
    reference that calibrates the PMC byte counters."""
    import torch

    from nlearn_amd import _lib
    from nlearn_amd.kernels.gemm import gemm_raw, padded_empty

    _lib.load()
    dev = torch.device("cuda:0")
    M, K, N = 16384, 512, 50257
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn((M, K), device=dev, generator=g).to(torch.bfloat16)
    w = padded_empty(K, N, torch.bfloat16, dev)
    w.copy_(torch.randn((K, N), device=dev, generator=g) * 0.02)
    y = padded_empty(M, N, torch.bfloat16, dev)
    dx = padded_empty(M, K, torch.bfloat16, dev)
    dw = padded_empty(K, N, torch.float32, dev)
    h = int(_traffic_products()[3][0].split("_")[2].split("x")[0])
    layer = []
    for kin, nout in ((512, 1536), (512, 512), (512, 2048), (2048, 512)):
        a = padded_empty(M, kin, torch.bfloat16, dev)
        a.copy_(torch.randn((M, kin), device=dev, generator=g))
        dy = padded_empty(M, nout, torch.bfloat16, dev)
        dy.copy_(torch.randn((M, nout), device=dev, generator=g))
        layer.append((a, dy, torch.empty((kin, nout), dtype=torch.float32, device=dev)))
    src = torch.ones(2**28, dtype=torch.float32, device=dev)   # 1 GiB
    dst = torch.empty_like(src)
    for _ in range(reps):
        gemm_raw(x, w, out=y)                 # logits = x W
        gemm_raw(y, w, "N", "T", out=dx)      # dX = dlogits W^T
        gemm_raw(x, y, "T", "N", out=dw)      # dW = x^T dlogits
        gemm_raw(x[:h], w, out=y[:h])         # the first of the step's two logits chunks
        for a, dy, out in layer:              # the layers' X^T dY
            gemm_raw(a, dy, "T", "N", out=out)
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"probe": "traffic", "products": [t for t, _ in _traffic_products()], "copy_bytes": 2**30,
                      "reps": reps}))


def _probe_dispatch_tags(names):
    """bench.py tags of the dispatches of --traffic-probe, given their kernel
    names in dispatch order: the GEMM kernels take the products' tags in launch
    order (cycling per repetition), a split-K reduction the tag of the GEMM
    before it, the 1 GiB copy "copy"; anything else (set-up) None."""
    order = [t for t, _ in _traffic_products()]
    tags, i, last = [], 0, None
    for n in names:
        if "copyBuffer" in n:
            tags.append("copy")
        elif "splitk_reduce_kernel" in n:
            tags.append(last)
        elif ("gemm2_kernel" in n or "gemm_persist_kernel" in n) and "<" in n:
            last = order[i % len(order)]
            i += 1
            tags.append(last)
        else:
            tags.append(None)
    return tags


def traffic_summary(fetch_dir: str, write_dir: str) -> None:
    """HBM bytes per launch of the probe's GEMMs from two rocprofv3 --pmc runs:
    each counter's median over the probe's repetitions, summed over the kernels
    of one product (a split product adds its reduction), scaled by what the
    same counter reads for the 1 GiB copy (known bytes)."""
    import csv
    import glob
    import statistics

    def read(d, counter):
        rows = []
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                if r["Counter_Name"] == counter:
                    rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"])))
        rows.sort()
        per = {}          # tag -> kernel name -> [KiB per dispatch]
        for (_, name, val), tag in zip(rows, _probe_dispatch_tags([r[1] for r in rows])):
            if tag:
                per.setdefault(tag, {}).setdefault(name, []).append(val)
        return {t: {k: statistics.median(v) for k, v in ks.items()} for t, ks in per.items()}

    fetch, write = read(fetch_dir, "FETCH_SIZE"), read(write_dir, "WRITE_SIZE")
    copy_bytes = 2 ** 30
    cf = sum(fetch["copy"].values())
    cw = sum(write["copy"].values())
    fs, ws = copy_bytes / (cf * 1024), copy_bytes / (cw * 1024)
    out = {"calibration": {"kernel": "__amd_rocclr_copyBuffer (torch copy_ of 1 GiB fp32)", "bytes": copy_bytes,
                           "fetch_kib_raw": cf, "write_kib_raw": cw, "fetch_scale": round(fs, 4),
                           "write_scale": round(ws, 4)},
           "commands": ["rocprofv3 --pmc FETCH_SIZE --kernel-trace --output-format csv -d <fetch> -o run -- "
                        "python3 <repo>/bench.py --traffic-probe",
                        "rocprofv3 --pmc WRITE_SIZE --kernel-trace --output-format csv -d <write> -o run -- "
                        "python3 <repo>/bench.py --traffic-probe",
                        "python3 bench.py --traffic-summary <fetch> <write>"],
           "kernels": {}}
    for tag, a in _traffic_products():
        fk, wk = sum(fetch.get(tag, {}).values()), sum(write.get(tag, {}).values())
        fb, wb = int(fk * 1024 * fs), int(wk * 1024 * ws)
        out["kernels"][tag] = {"dispatch_kernels": sorted(fetch.get(tag, {})), "fetch_kib_raw": fk,
                               "write_kib_raw": wk, "fetch_bytes": fb, "write_bytes": wb,
                               "per_kernel_fetch_kib_raw": fetch.get(tag, {}),
                               "per_kernel_write_kib_raw": write.get(tag, {}),
                               "bytes_per_launch": fb + wb, "algorithmic_bytes": a,
                               "traffic_over_algorithmic": round((fb + wb) / a, 3)}
    with open(TRAFFIC_FILE, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps({k: v["bytes_per_launch"] for k, v in out["kernels"].items()}))


BUSY_FIRST_KERNEL = "embed_fwd_kernel"   # launched once per step, at its start (the embedding lookup)


def _kernel_short_name(name: str) -> str:
    """A demangled kernel name without namespaces, ``void`` and the argument
    list (template arguments kept, so tile configurations stay distinct)."""
    name = name.replace("(anonymous namespace)::", "").replace("nl::", "").replace("void ", "")
    return name.split("(")[0][:110]


def busy_summary(trace_dir: str, steps: int, bs: int, seq: int) -> None:
    """Busy ratio of the graphed step from a rocprofv3 kernel trace of
    --replay-probe: the last ``steps`` step starts (each step's first kernel)
    delimit the replays; over that window, the union of all kernel intervals
    (overlapping kernels counted once) over the wall time, plus the plain sum
    of kernel durations (which exceeds the union where streams overlap) and
    the per-kernel time per step."""
    import csv
    import glob

    rows = []
    for f in glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]))
    out = busy_stats(rows, steps, bs, seq)
    path = os.path.join(os.path.dirname(TRAFFIC_FILE), f"busy_bs{bs}_seq{seq}.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps({k: out[k] for k in ("wall_ms_per_step", "busy_union_ms_per_step", "busy_ratio",
                                          "kernel_sum_over_wall")}))


def trace_summary(trace_dir: str, out_md: str, title: str, command: str, steps: int,
                  bench_json: str | None = None, kernel: str | None = None) -> None:
    """Markdown table of a rocprofv3 --kernel-trace (csv) run: per kernel, the
    dispatches, time per step (``steps`` = steps the profiled command ran) and
    the mean, median, min and max duration. With the bench line the profiled
    run printed and the dominant kernel's name, the line's HIP-event mean is
    set beside the kernel's rocprof mean."""
    import csv
    import glob
    import statistics

    rows = []
    for f in glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]))
    per = defaultdict(list)
    for a, b, n in sorted(rows):
        per[_kernel_short_name(n)].append((b - a) / 1e3)
    total = sum(sum(v) for v in per.values())
    lines = [f"# {title}", "", "Command (repository root of the GPU host, `TMPDIR=/tmp`):", "", "```", command, "```",
             "", f"Kernel time of all {steps} steps the command runs (warm-up, timed, and bench.py's per-kernel "
             f"passes): {total / steps / 1e3:.3f} ms per step.", ""]
    if bench_json and kernel:
        with open(bench_json) as f:
            line = json.loads([l for l in f if l.startswith("{")][-1])
        roof = line["roofline"]
        d = per.get(kernel, [])
        if d:
            mean = statistics.mean(d)
            lines += [f"Dominant kernel `{kernel}` (bench tag `{roof['kernel']}`): rocprof mean {mean:.1f} us over "
                      f"{len(d)} dispatches (median {statistics.median(d):.1f}); the bench line of this run: "
                      f"{roof['avg_us']:.1f} us in the step (frac {roof['frac']}), {roof['avg_us_isolated']:.1f} us "
                      f"alone (frac {roof['frac_isolated']}), {line['ms_per_step']} ms per step, "
                      f"{line['value'] / 1e6:.3f} M tokens/s.", ""]
            # the same dispatches split by bench.py's passes, in launch order
            lps = int(round(line["detail"]["kernels_in_step"][roof["kernel"]]["launches_per_step"]))
            K, W = line["steps"], line["warmup"]
            passes = [("warm-up and capture", max(W, 3)), ("timed graph replays", K),
                      ("in-step pass (bench HIP events)", K), ("one-stream pass (alone)", min(K, 5))]
            if "variant_bs4_seq4096" in line["detail"]:
                vk, vw = min(K, 20), min(W, 5)
                passes += [("variant warm-up", max(vw, 3)), ("variant replays", vk), ("variant in-step pass", vk),
                           ("variant alone", min(vk, 5))]
            if sum(n for _, n in passes) * lps == len(d):
                lines += ["| pass | dispatches | rocprof mean us |", "|---|---:|---:|"]
                i = 0
                for name, n in passes:
                    seg = d[i:i + n * lps]
                    i += n * lps
                    lines.append(f"| {name} | {len(seg)} | {statistics.mean(seg):.1f} |")
                lines.append("")
    lines += ["| ms / step | calls / step | mean us | median us | min us | max us | kernel |",
              "|---:|---:|---:|---:|---:|---:|---|"]
    for k, d in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        if sum(d) / steps < 1.0:   # below 1 us per step
            continue
        lines.append(f"| {sum(d) / steps / 1e3:.3f} | {len(d) / steps:.2f} | {statistics.mean(d):.1f} | "
                     f"{statistics.median(d):.1f} | {min(d):.1f} | {max(d):.1f} | `{k}` |")
    with open(out_md, "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines[:14]))


def busy_stats(rows, steps: int, bs: int, seq: int) -> dict:
    """The busy_summary figures from (start_ns, end_ns, kernel_name) rows."""
    rows = sorted(rows)
    starts = [t0 for t0, _, name in rows if BUSY_FIRST_KERNEL in name]
    if len(starts) < steps + 1:
        raise SystemExit(f"busy-summary: found {len(starts)} step starts, need {steps + 1}")
    # the window: from the first of the last `steps` step starts to the last kernel's end
    w0 = starts[-steps]
    win = [(a, b, n) for a, b, n in rows if a >= w0]
    w1 = max(b for _, b, _ in win)
    union, cur0, cur1 = 0, None, None
    for a, b, _ in win:
        if cur1 is None or a > cur1:
            if cur1 is not None:
                union += cur1 - cur0
            cur0, cur1 = a, b
        else:
            cur1 = max(cur1, b)
    union += cur1 - cur0
    total = sum(b - a for a, b, _ in win)
    per = defaultdict(lambda: [0, 0])
    for a, b, n in win:
        short = _kernel_short_name(n)
        per[short][0] += b - a
        per[short][1] += 1
    wall = w1 - w0
    out = {"workload": f"train_step fwd+bwd+AdamW d512/8h/4L vocab50257 bs{bs} seq{seq}, hip_graph replays",
           "command": f"rocprofv3 --kernel-trace --output-format csv -d <dir> -o run -- python3 bench.py "
                      f"--replay-probe --steps {steps} --batch-size {bs} --seq-len {seq}; "
                      f"python3 bench.py --busy-summary <dir> --steps {steps} --batch-size {bs} --seq-len {seq}",
           "replays": steps, "wall_ms_per_step": round(wall / steps / 1e6, 4),
           "busy_union_ms_per_step": round(union / steps / 1e6, 4),
           "busy_ratio": round(union / wall, 4),
           "kernel_sum_ms_per_step": round(total / steps / 1e6, 4),
           "kernel_sum_over_wall": round(total / wall, 4),
           "kernels_ms_per_step": {k: {"ms": round(v[0] / steps / 1e6, 4), "calls": round(v[1] / steps, 2)}
                                   for k, v in sorted(per.items(), key=lambda kv: -kv[1][0])}}
    return out


def flash_probe(n: int, S: int, reps: int = 5) -> None:
    """BASELINE configs[1] flash forward and backward at (n, S, 64), bf16
    N(0,1) inputs, ``reps`` times each: the preprocess, dK/dV and dQ kernels
    run as in nl_flash_attention_bwd (one stream)."""
    import torch

    from nlearn_amd import _lib
    from nlearn_amd.attention import flash_bwd_raw4, flash_fwd_raw4

    _lib.load()
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    q, k, v, do = (torch.randn((n // 8, 8, S, 64), generator=g, device=dev).to(torch.bfloat16) for _ in range(4))
    for _ in range(reps):
        O, L = flash_fwd_raw4(q, k, v)
        flash_bwd_raw4(q, k, v, O, do, L)
    torch.cuda.synchronize()
    print(json.dumps({"probe": "flash", "shape": [n, S, 64], "reps": reps}))


def pmc_summary(out_md: str, title: str, dirs) -> None:
    """Median of every counter per kernel over the dispatches in the rocprofv3
    --pmc CSV output of ``dirs`` (one directory per counter pass), as a
    markdown table, with the derived ratios used in the design notes:
    MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 x CUs x 4 SIMDs)
    (rocprofv3 sums GRBM_GUI_ACTIVE over the 8 XCDs, and the MFMA busy cycles
    over every SIMD; this reproduces flops / (time x peak) at the measured clock),
    VALU instructions per MFMA, LDS bank conflicts per LDS active cycle."""
    import csv
    import glob
    import statistics

    per = defaultdict(lambda: defaultdict(list))
    for d in dirs:
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                if "nl::" not in r["Kernel_Name"]:
                    continue
                name = _kernel_short_name(r["Kernel_Name"])
                per[name][r["Counter_Name"]].append(float(r["Counter_Value"]))
    cus = 256
    lines = [f"# {title}", "", "Medians over the dispatches of each kernel (rocprofv3 --pmc, one pass per "
             "counter set). MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 XCDs x 256 CUs x 4 "
             "SIMDs); LDS conflict = SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE; cycles = GRBM_GUI_ACTIVE / 8.",
             ""]
    counters = sorted({c for k in per.values() for c in k})
    lines.append("| kernel | cycles | MFMA busy | VALU / MFMA | LDS / MFMA | LDS conflict | "
                 + " | ".join(counters) + " |")
    lines.append("|---|---:|---:|---:|---:|---:|" + "---:|" * len(counters))
    for name, cs in sorted(per.items()):
        med = {c: statistics.median(v) for c, v in cs.items()}
        busy = med.get("SQ_VALU_MFMA_BUSY_CYCLES", 0) / (med["GRBM_GUI_ACTIVE"] / 8 * cus * 4) \
            if med.get("GRBM_GUI_ACTIVE") else float("nan")
        vpm = med["SQ_INSTS_VALU"] / med["SQ_INSTS_MFMA"] if med.get("SQ_INSTS_MFMA") else float("nan")
        conf = med["SQ_LDS_BANK_CONFLICT"] / med["SQ_LDS_IDX_ACTIVE"] if med.get("SQ_LDS_IDX_ACTIVE") else float("nan")
        lpm = med["SQ_INSTS_LDS"] / med["SQ_INSTS_MFMA"] if med.get("SQ_INSTS_MFMA") else float("nan")
        cyc = med.get("GRBM_GUI_ACTIVE", float("nan")) / 8
        lines.append(f"| `{name[:60]}` | {cyc:.0f} | {busy:.3f} | {vpm:.2f} | {lpm:.2f} | {conf:.3f} | "
                     + " | ".join(f"{med[c]:.4g}" if c in med else "" for c in counters) + " |")
    with open(out_md, "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))


def load_busy(bs: int, seq: int):
    """The committed busy-ratio summary of this workload, if any."""
    try:
        with open(os.path.join(os.path.dirname(TRAFFIC_FILE), f"busy_bs{bs}_seq{seq}.json")) as f:
            b = json.load(f)
        return {"busy_ratio": b["busy_ratio"], "wall_ms_per_step": b["wall_ms_per_step"],
                "source": f"profiles/busy_bs{bs}_seq{seq}.json (rocprofv3 kernel trace of graph replays)"}
    except (OSError, ValueError, KeyError):
        return None


def load_traffic(tag: str):
    """HBM bytes per launch of `tag` from the committed PMC summary, if it covers it."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    k = t.get("kernels", {}).get(tag)
    return k.get("bytes_per_launch") if k else None


def _median_us(fn, n: int = 50, batches: int = 5, warmup: int = 5) -> float:
    """Kernel-level timing: ``warmup`` untimed calls, then ``batches`` runs of
    ``n`` back-to-back calls, each bracketed by HIP events on the current
    stream; the median of the per-call means, in microseconds."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    means = []
    for _ in range(batches):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        means.append(e0.elapsed_time(e1) / n * 1e3)
    return float(sorted(means)[len(means) // 2])


def gemm_compare(reps: int = 50) -> None:
    """The BASELINE GEMM products (configs[2]: M = 16384 and the model's (K, N),
    each as forward NN, dX = dY.W^T (NT) and dW = X^T.dY (TN)) through this
    library and through torch.matmul (hipBLASLt), both timed by ``_median_us``
    (median of 5 batches of ``reps`` calls after 5 warm-ups). One JSON line per
    product. torch's dW comes out in bf16, ours in fp32 as the training step
    uses it."""
    import torch

    from nlearn_amd.kernels.gemm import gemm_raw, padded_empty

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    M = 16384

    for K, N in ((512, 1536), (512, 512), (512, 2048), (2048, 512), (512, 50257)):
        X = torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16)
        W = padded_empty(K, N, torch.bfloat16, dev)
        W.copy_(torch.randn((K, N), generator=g, device=dev) * 0.05)
        dY = padded_empty(M, N, torch.bfloat16, dev)
        dY.copy_(torch.randn((M, N), generator=g, device=dev))
        Y, dX = padded_empty(M, N, torch.bfloat16, dev), padded_empty(M, K, torch.bfloat16, dev)
        dW = padded_empty(K, N, torch.float32, dev)
        for lay, ours, lib in (("NN", lambda: gemm_raw(X, W, out=Y), lambda: X @ W),
                               ("NT", lambda: gemm_raw(dY, W, "N", "T", out=dX), lambda: dY @ W.t()),
                               ("TN", lambda: gemm_raw(X, dY, "T", "N", out=dW), lambda: X.t() @ dY)):
            mm, nn, kk = (M, N, K) if lay == "NN" else (M, K, N) if lay == "NT" else (K, N, M)
            t_ours, t_lib = _median_us(ours, reps), _median_us(lib, reps)
            fl = 2.0 * mm * nn * kk
            print(json.dumps({"gemm": f"{lay}_{mm}x{nn}x{kk}", "ours_us": round(t_ours, 1),
                              "hipblaslt_us": round(t_lib, 1), "ours_tflops": round(fl / t_ours / 1e6, 1),
                              "hipblaslt_tflops": round(fl / t_lib / 1e6, 1),
                              "speedup": round(t_lib / t_ours, 3)}), flush=True)


def kernel_configs(reps: int = 50) -> None:
    """BASELINE configs[1] (causal flash forward and backward at (256, 512, 64)
    and (32, 4096, 64), head dim 64, scale 1/8) and configs[3] (CE + dlogits at
    (16384, 50257), logits ~ N(0, 2) bf16) in isolation: this library against
    torch's own kernels for the same work (scaled_dot_product_attention with
    is_causal, and cross_entropy forward + backward), timed by ``_median_us``
    (median of 5 batches of ``reps`` calls after 5 warm-ups). One JSON line per
    case with the roofline fraction."""
    import torch

    from nlearn_amd.attention import flash_bwd_raw4, flash_fwd_raw4
    from nlearn_amd.kernels.cross_entropy import ce_fwd_bwd_raw

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)

    def timeit(fn, n=reps):
        return _median_us(fn, n)

    for n, S in ((256, 512), (32, 4096)):
        B, H = n // 8, 8
        q, k, v, do = (torch.randn((B, H, S, 64), generator=g, device=dev).to(torch.bfloat16) for _ in range(4))
        O, L = flash_fwd_raw4(q, k, v)
        f = 2.0 * n * S * S * 64  # causal forward: QK^T and PV over the lower triangle
        t_f = timeit(lambda: flash_fwd_raw4(q, k, v))
        t_b = timeit(lambda: flash_bwd_raw4(q, k, v, O, do, L))
        qr, kr, vr = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
        sdpa = torch.nn.functional.scaled_dot_product_attention
        t_tf = timeit(lambda: sdpa(qr, kr, vr, is_causal=True))
        out = sdpa(qr, kr, vr, is_causal=True)
        t_tb = timeit(lambda: torch.autograd.grad(out, (qr, kr, vr), do, retain_graph=True))
        for tag, t_o, t_t, w in (("fwd", t_f, t_tf, f), ("bwd", t_b, t_tb, 2.5 * f)):
            print(json.dumps({"case": f"flash_{tag}_{n}x{S}x64", "ours_us": round(t_o, 1), "torch_us": round(t_t, 1),
                              "ours_frac": round(w / t_o / 1e6 / PEAK_BF16_TFLOPS, 4),
                              "torch_frac": round(w / t_t / 1e6 / PEAK_BF16_TFLOPS, 4),
                              "speedup": round(t_t / t_o, 3)}), flush=True)
    M, V = 16384, 50257
    logits = (torch.randn((M, V), generator=g, device=dev) * 2.0).to(torch.bfloat16)
    t = torch.randint(0, V, (M,), generator=g, device=dev)
    t_o = timeit(lambda: ce_fwd_bwd_raw(logits, t))
    lr = logits.detach().clone().requires_grad_(True)

    def torch_ce():
        loss = torch.nn.functional.cross_entropy(lr, t)
        return torch.autograd.grad(loss, lr)

    t_t = timeit(torch_ce)
    byt = 4.0 * M * V + 12.0 * M
    print(json.dumps({"case": f"ce_fwd_bwd_{M}x{V}", "ours_us": round(t_o, 1), "torch_us": round(t_t, 1),
                      "ours_frac": round(byt / t_o / 1e3 / PEAK_HBM_GBS, 4),
                      "torch_frac": round(byt / t_t / 1e3 / PEAK_HBM_GBS, 4), "speedup": round(t_t / t_o, 3)}),
          flush=True)
    # what the box sustains for plain traffic: a 2 GiB device copy (read + write), fill (write), sum (read)
    del logits, lr
    n = 2 * 2**30 // 4
    src = torch.randn(n, generator=g, device=dev)
    dst = torch.empty_like(src)
    for tag, fn, byt in (("hbm_copy_2GiB", lambda: dst.copy_(src), 8.0 * n), ("hbm_fill_2GiB", lambda: dst.fill_(1.0), 4.0 * n),
                         ("hbm_sum_2GiB", lambda: src.sum(), 4.0 * n)):
        t_x = timeit(fn)
        print(json.dumps({"case": tag, "torch_us": round(t_x, 1), "tbs": round(byt / t_x / 1e6, 3),
                          "torch_frac": round(byt / t_x / 1e3 / PEAK_HBM_GBS, 4)}), flush=True)


def torch_step(bs: int, seq: int, steps: int, warmup: int) -> None:
    """The same training step (BASELINE model, bs x seq tokens, AdamW) written
    with plain PyTorch ops on the same GPU: bf16 weights and activations with
    fp32 master weights in torch.optim.AdamW(fused=True), F.layer_norm, bf16
    matmuls (hipBLASLt), scaled_dot_product_attention(is_causal=True), tanh
    GELU, F.cross_entropy. Eager launches, timed like the main step. A
    reference point for what the library buys over idiomatic PyTorch; prints
    one JSON line."""
    import torch
    import torch.nn.functional as F

    from nlearn_amd.model import ModelConfig, init_params_numpy, tree_leaves, tree_map

    dev = torch.device("cuda:0")
    cfg = ModelConfig(max_seq_len=max(512, seq))
    params = tree_map(lambda a_: torch.from_numpy(a_).to(dev).requires_grad_(True), init_params_numpy(0, cfg))
    opt = torch.optim.AdamW(tree_leaves(params), lr=1e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1,
                            fused=True)
    H, dh = cfg.n_heads, cfg.d_head
    bf = torch.bfloat16

    def loss_fn(batch):
        ids, tgt = batch[:, :-1], batch[:, 1:]
        e = params["embeddings"]
        x = (e["token_embed"][ids] + e["pos_embed"][:seq]).to(bf)
        for p in params["blocks"]:
            h = F.layer_norm(x, (cfg.d_model,), p["ln1"]["gamma"].to(bf), p["ln1"]["beta"].to(bf), cfg.ln_eps)
            qkv = (h @ p["attn"]["W_qkv"].to(bf)).view(bs, seq, 3, H, dh).permute(2, 0, 3, 1, 4)
            a_ = F.scaled_dot_product_attention(qkv[0], qkv[1], qkv[2], is_causal=True)
            x = x + a_.transpose(1, 2).reshape(bs, seq, cfg.d_model) @ p["attn"]["W_o"].to(bf)
            h = F.layer_norm(x, (cfg.d_model,), p["ln2"]["gamma"].to(bf), p["ln2"]["beta"].to(bf), cfg.ln_eps)
            f = p["ffn"]
            u = F.gelu(h @ f["W1"].to(bf) + f["b1"].to(bf), approximate="tanh")
            x = x + u @ f["W2"].to(bf) + f["b2"].to(bf)
        lf = params["ln_final"]
        x = F.layer_norm(x, (cfg.d_model,), lf["gamma"].to(bf), lf["beta"].to(bf), cfg.ln_eps)
        logits = x @ params["lm_head"].to(bf)
        return F.cross_entropy(logits.view(-1, cfg.vocab_size).float(), tgt.reshape(-1).long())

    g = torch.Generator(device=dev).manual_seed(0)
    batches = [torch.randint(0, cfg.vocab_size, (bs, seq + 1), generator=g, device=dev) for _ in range(4)]

    def step(b):
        opt.zero_grad(set_to_none=True)
        loss = loss_fn(b)
        loss.backward()
        opt.step()
        return loss

    for i in range(warmup):
        step(batches[i % 4])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        loss = step(batches[i % 4])
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    print(json.dumps({"torch_step": f"d512/8h/4L vocab50257 bs{bs} seq{seq}", "ms_per_step": round(dt / steps * 1e3, 3),
                      "tokens_per_s": round(bs * seq * steps / dt, 1), "final_loss": round(float(loss.detach()), 4),
                      "peak_hbm_gib": round(torch.cuda.max_memory_allocated() / 2**30, 2)}), flush=True)


def main():
    a = _args()
    if a.torch_step:
        torch_step(a.batch_size, a.seq_len, a.steps, a.warmup)
        return
    if a.traffic_probe:
        traffic_probe()
        return
    if a.gemm_compare:
        gemm_compare()
        return
    if a.kernel_configs:
        kernel_configs()
        return
    if a.traffic_summary:
        traffic_summary(*a.traffic_summary)
        return
    if a.trace_summary:
        t = a.trace_summary
        trace_summary(t[0], t[1], t[2], t[3], int(t[4]), *(t[5:7]))
        return
    if a.busy_summary:
        busy_summary(a.busy_summary, a.steps, a.batch_size, a.seq_len)
        return
    if a.flash_probe:
        flash_probe(*a.flash_probe)
        return
    if a.pmc_summary:
        pmc_summary(a.pmc_summary[0], a.pmc_summary[1], a.pmc_summary[2:])
        return
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the data-parallel step would all-reduce "
              "the gradients over RCCL before AdamW). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch

    from nlearn_amd import _lib

    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        sys.exit(1)
    _lib.load()
    dev = torch.device("cuda:0")
    bs, seq = a.batch_size, a.seq_len
    graph = not a.no_graph
    if a.replay_probe:
        run_workload(torch, dev, bs, seq, a.steps, a.warmup, graph, a.fused_lmhead, replay_only=True)
        return
    r = run_workload(torch, dev, bs, seq, a.steps, a.warmup, graph, a.fused_lmhead)
    kernels, iso = r["kernels"], r["iso"]
    dom_tag = dominant_kernel(kernels, iso)
    roof = None
    if dom_tag:
        k = kernels[dom_tag]
        roof = {"bound": k["bound"], "achieved": round(k["achieved"], 2), "peak": k["peak"], "unit": k["unit"],
                "frac": round(k["frac"], 4), "traffic": load_traffic(dom_tag), "kernel": dom_tag,
                "avg_us": round(k["avg_us"], 2),
                "chosen_by": "largest time per step with every kernel alone on the GPU (one-stream pass)",
                "timing": "in the step: HIP events on the launch stream, two-stream overlap as in the replays",
                "frac_isolated": round(iso[dom_tag]["frac"], 4) if dom_tag in iso else None,
                "avg_us_isolated": round(iso[dom_tag]["avg_us"], 2) if dom_tag in iso else None}

    out = {
        "metric": "train tokens/sec d512/4L/seq512 bs32 (1 GPU)",
        "value": round(r["value"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(r["ms"], 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic uniform tokens, random-init weights (seeded)",
        "config": {"workload": f"train_step fwd+bwd+AdamW d512/8h/4L vocab50257 bs{bs} seq{seq}",
                   "global_batch": bs, "seq_len": seq, "parallelism": "single-gpu",
                   "launch": "hip_graph" if graph else "eager",
                   "loss": "linear_cross_entropy" if a.fused_lmhead else "linear+cross_entropy"},
        "roofline": roof,
        "cpu_baseline": None,
        "detail": {
            "mfu_matmul": r["mfu"],
            "matmul_tflop_per_step": r["tflop"],
            "six_n_t_tflops": r["six_n_t_tflops"],
            "peak_hbm_gib": r["peak_hbm_gib"],
            "busy": load_busy(bs, seq),
            "final_loss": r["loss"],
            "kernels_in_step": _table(kernels),
            "kernels_isolated": _table(iso),
        },
    }
    del r
    # BASELINE configs[4] also asks for the bs4 x seq4096 variant: the same step,
    # timed the same way in the same process (after the headline's buffers are
    # freed, so its peak memory is its own)
    if not a.no_variant and (bs, seq) != VARIANT:
        out["detail"]["variant_bs4_seq4096"] = variant_detail(torch, dev, a.steps, a.warmup, graph, a.fused_lmhead)
    if not a.no_cpu_baseline:
        try:
            out["cpu_baseline"] = cpu_baseline(a.cpu_seconds)
        except ImportError as e:  # oracle absent from the tree
            out["cpu_baseline"] = {"error": str(e)}
    print(json.dumps(out))


def variant_detail(torch, dev, steps: int, warmup: int, graph: bool, fused) -> dict:
    """BASELINE configs[4]'s second workload (bs4 x seq4096) timed like the
    headline: tokens/s, MFU, peak HBM, busy ratio and its dominant kernel. A
    failure is reported in the result, so the headline line is still printed."""
    vb, vs = VARIANT
    try:
        v = run_workload(torch, dev, vb, vs, min(steps, 20), min(warmup, 5), graph, fused)
    except (RuntimeError, MemoryError) as e:
        return {"error": f"{type(e).__name__}: {e}"}
    vdom = dominant_kernel(v["kernels"], v["iso"])
    return {
        "workload": f"train_step fwd+bwd+AdamW d512/8h/4L vocab50257 bs{vb} seq{vs}",
        "tokens_per_s": round(v["value"], 1), "ms_per_step": round(v["ms"], 3), "steps": v["steps"],
        "mfu_matmul": v["mfu"], "matmul_tflop_per_step": v["tflop"], "peak_hbm_gib": v["peak_hbm_gib"],
        "busy": load_busy(vb, vs), "final_loss": v["loss"],
        "dominant_kernel": None if vdom is None else {
            "kernel": vdom, "chosen_by": "largest time per step alone on the GPU",
            "frac": round(v["kernels"][vdom]["frac"], 4), "avg_us": round(v["kernels"][vdom]["avg_us"], 2),
            "frac_isolated": round(v["iso"][vdom]["frac"], 4),
            "avg_us_isolated": round(v["iso"][vdom]["avg_us"], 2)},
        "kernels_isolated": _table(v["iso"]),
    }


# BASELINE configs[4]'s second workload
VARIANT = (4, 4096)


def _table(kk):
    return {k: {kk2: (round(vv, 4) if isinstance(vv, float) else vv) for kk2, vv in v.items()}
            for k, v in sorted(kk.items(), key=lambda kv: -kv[1]["time_per_step_ms"])}


def dominant_kernel(kernels: dict, iso: dict):
    """The kernel with the largest time per step when every kernel runs alone
    (the one-stream pass): in the overlapped pass a kernel sharing CUs with the
    other stream looks longer than it is. Falls back to the overlapped pass."""
    src = {k: v for k, v in iso.items() if k in kernels} or kernels
    return max(src, key=lambda k: src[k]["time_per_step_ms"]) if src else None


def run_workload(torch, dev, bs: int, seq: int, steps: int, warmup: int, graph: bool, fused: bool,
                 replay_only: bool = False):
    """One training workload: warm-up (and capture), ``steps`` timed steps,
    then the per-kernel passes (overlapped as in the step, and one-stream);
    returns the figures and frees every buffer it made."""
    import gc

    from nlearn_amd import _lib
    from nlearn_amd.model import ModelConfig, flops_per_step, init_model
    from nlearn_amd.train import AdamW, SyntheticTokens, make_train_step, warmup_cosine_decay_schedule

    gc.collect()
    torch.cuda.empty_cache()
    # peak memory of this workload alone: parameters, optimizer state, the
    # eager warm-up steps, the capture and the timed steps
    torch.cuda.reset_peak_memory_stats()
    cfg = ModelConfig(max_seq_len=max(512, seq))
    params = init_model(0, cfg, dev)
    total_updates = warmup + steps
    opt = AdamW(warmup_cosine_decay_schedule(0.0, 1e-3, 200, max(total_updates, 1000), 1e-4))
    state = opt.init(params)
    probe = KernelProbe(torch)
    _lib.set_probe(probe)
    step = make_train_step(opt, cfg, graph=graph, warmup=2, fused_lmhead=fused)
    data = SyntheticTokens(bs, seq, cfg.vocab_size, seed=0, device=dev)
    batches = [data.get_batch() for _ in range(4)]

    # warm-up (in graph mode the step is captured during it and replayed)
    for i in range(max(warmup, 3 if graph else 0)):
        params, state, loss = step(params, state, batches[i % 4])
    torch.cuda.synchronize()
    if replay_only:
        for i in range(steps):
            params, state, loss = step(params, state, batches[i % 4])
        torch.cuda.synchronize()
        _lib.set_probe(None)
        print(json.dumps({"probe": "replay", "steps": steps, "loss": round(float(loss), 4)}))
        return None

    probe.enabled = not graph
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        params, state, loss = step(params, state, batches[i % 4])
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    peak = torch.cuda.max_memory_allocated()
    eager = None
    if graph:
        # Per-kernel durations: events cannot be placed between the nodes of a
        # replayed graph (torch-ROCm refuses external events in a capture), so
        # the same step runs `steps` more times eagerly, every kernel bracketed
        # by events on its launch stream; kernels, shapes and the two-stream
        # overlap are those of the replays.
        eager = make_train_step(opt, cfg, graph=False, fused_lmhead=fused)
        probe.enabled = True
        for i in range(steps):
            params, state, loss = eager(params, state, batches[i % 4])
        torch.cuda.synchronize()
    probe.enabled = False
    # The same step once more on one stream (no weight-gradient overlap): every
    # kernel alone on the GPU, its own speed without CUs shared with the other
    # stream.
    iso_probe = KernelProbe(torch)
    _lib.set_probe(iso_probe)
    solo = make_train_step(opt, cfg, graph=False, fused_lmhead=fused, overlap_wgrad=False)
    iso_steps = min(steps, 5)
    iso_probe.enabled = True
    for i in range(iso_steps):
        params, state, loss = solo(params, state, batches[i % 4])
    torch.cuda.synchronize()
    iso_probe.enabled = False
    _lib.set_probe(None)
    fl = flops_per_step(cfg, bs, seq)
    res = {"value": bs * seq * steps / dt, "ms": dt / steps * 1e3, "steps": steps,
           "kernels": probe.summary(steps), "iso": iso_probe.summary(iso_steps),
           "mfu": round(fl["total"] / (dt / steps) / (PEAK_BF16_TFLOPS * 1e12), 4),
           "tflop": round(fl["total"] / 1e12, 4),
           "six_n_t_tflops": round(fl["six_n_t"] / (dt / steps) / 1e12, 2),
           "peak_hbm_gib": round(peak / 2**30, 2), "loss": round(float(loss.detach()), 4)}
    del params, state, step, eager, solo, batches, loss, opt, probe, iso_probe
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return res


if __name__ == "__main__":
    main()
