"""Text summaries of rocprofv3 CSV output for the 1024x1024 denoise benchmark.

    trace   DIR [--steps K] [--command CMD]
        from DIR/*_kernel_trace.csv (rocprofv3 --kernel-trace --stats -f csv): the
        per-kernel table and, over the last K Euler steps of the run (the timed steps
        of bench.py), the device busy / idle split and the largest gaps between
        consecutive kernels.
    traffic FETCH_DIR WRITE_DIR --sources-sha256 H [--command CMD ...]
        from two rocprofv3 --pmc runs (FETCH_SIZE, then WRITE_SIZE) of
        bench.py --copy-calibration-mib N: HBM bytes per dispatch of each kernel,
        scaled by what each counter reads for the plain copy kernel, and per launch
        of each block stage (bench.py's kernel classes), closed by a ```json traffic```
        record that bench.py reads for its roofline.
    mfma    DIR
        from one rocprofv3 --pmc run with SQ_BUSY_CU_CYCLES SQ_VALU_MFMA_BUSY_CYCLES
        SQ_INSTS_VALU SQ_INSTS_MFMA SQ_INSTS_LDS GRBM_GUI_ACTIVE: per kernel, the clock
        it ran at, the matrix cores' busy fraction and VALU / LDS instructions per MFMA.

Writes Markdown to stdout, or to --output FILE. Each summary states the commands that
made it: the profiler runs given with --command, then this tool's own invocation.
Reads only the CSV files it is given.
"""
import argparse
import csv
import json
import shlex
import statistics
import sys
from collections import defaultdict
from pathlib import Path

# Kernel-name fragments -> short names, first match wins.
SHORT = [
    ("split_reduce_kernelIDF16_Li2", "reduce(up/gate)"), ("split_reduce_kernelIDF16_Li0", "reduce(qkv)"),
    ("split_reduce_kernelIu6__bf16S", "reduce(bf16)"),
    ("split_reduce_kernel<float, 1", "reduce(gate-resid)"), ("split_reduce_kernel<float, 0", "reduce(f32)"),
    ("pingpong6kernelIDF16_DF16_Li5", "gemm qkv+norm+rope"), ("pingpong6kernelIDF16_DF16_Li2", "gemm up/gate+geglu"),
    ("pingpong6kernelIDF16_fLi1", "gemm gate-resid"), ("pingpong6kernelIDF16_DF16_Li0", "gemm store"),
    ("pingpong6kernelIDF16_fLi0", "gemm f32 out"), ("pingpong6kernelIDF16_DF16_Li4", "gemm up/gate+swiglu"),
    ("split_reduce_kernelIDF16_Li4", "reduce(up/gate swiglu)"), ("rmsnorm_persist", "rmsnorm (row-major)"),
    ("sdl6kernel", "sdpa"), ("sdl14combine", "sdpa combine"),
    ("rmsnorm_pair_k32", "rmsnorm+modulate"), ("qk_rope_permuted", "qk norm+rope (split tail)"),
    ("qk_norm_rope", "qk norm+rope"), ("euler", "euler"), ("finite", "finite"), ("fill_int", "fill_int"),
    ("copyBuffer", "copy"), ("gemv", "gemv"), ("layernorm", "layernorm+mod"), ("transpose_tokens", "to tokens"),
    ("tokens_latent", "to latent"), ("convert_kernel", "convert/copy"), ("normal_kernel", "normal init"),
    ("tile_k32", "k32 tiling"),
]


def invocation():
    """This tool's command line as run from the repository root."""
    script = Path(__file__).resolve()
    try:
        script = script.relative_to(Path.cwd().resolve())
    except ValueError:
        pass
    return " ".join(["python3", shlex.quote(str(script)), *map(shlex.quote, sys.argv[1:])])


def commands(args):
    """The profiler runs (--command) and then the summary's own invocation."""
    return [*args.command, invocation()]


def emit(args, lines):
    text = "\n".join(lines) + "\n"
    if getattr(args, "output", None):
        Path(args.output).write_text(text)
    else:
        sys.stdout.write(text)


def short(name):
    for key, val in SHORT:
        if key in name:
            return val
    return name[:60]


def stage_of(name, previous):
    """(block stage, main) of a dispatch: the stage is bench.py's kernel class, given the
    previous dispatch's stage (the out and down projections share a kernel and are told
    apart by what ran before them, the SDPA or the up/gate GEMM); `main` is False for the
    split-K reductions, SDPA combines and split-tail passes that finish a stage's launch."""
    s = short(name)
    stages = {"rmsnorm+modulate": "rmsnorm_modulate", "gemm qkv+norm+rope": "gemm_qkv", "gemm store": "gemm_qkv",
              "qk norm+rope": "qk_norm_rope", "sdpa": "sdpa", "gemm up/gate+geglu": "gemm_up_gate"}
    if s in stages:
        return stages[s], True
    if s == "gemm gate-resid":
        return ("gemm_out" if previous == "sdpa" else "gemm_down"), True
    finishing = {"reduce(qkv)": "gemm_qkv", "qk norm+rope (split tail)": "gemm_qkv", "sdpa combine": "sdpa",
                 "reduce(up/gate)": "gemm_up_gate",
                 "reduce(gate-resid)": previous if previous in ("gemm_out", "gemm_down") else None}
    return finishing.get(s), False


def read_csv(directory, suffix):
    files = sorted(Path(directory).rglob(f"*{suffix}"))
    if not files:
        sys.exit(f"no *{suffix} under {directory}")
    rows = []
    for f in files:
        with open(f, newline="") as fh:
            rows += list(csv.DictReader(fh))
    return rows


def bench_classes(log):
    """The HIP-event class table of the last bench.py JSON line in a log."""
    line = [x for x in Path(log).read_text().splitlines() if x.startswith("{")][-1]
    d = json.loads(line)
    out = ["", "HIP-event figures of the same run (per launch of each class, split-K reduction included):", "",
           "| class | launches | avg us | TFLOP/s |", "|---|---:|---:|---:|"]
    for name, k in d["kernels"].items():
        tf = "-" if k.get("tflops") is None else f"{k['tflops']:.1f}"
        out.append(f"| {name} | {k['launches']} | {k['avg_us']:.1f} | {tf} |")
    out += ["", f"{d['value']:.2f} {d['unit']}, {d['ms_per_step']:.2f} ms per step under the profiler."]
    return out


def trace(args):
    rows = read_csv(args.dir, "_kernel_trace.csv")
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    dur = defaultdict(list)
    for r in rows:
        dur[r["Kernel_Name"]].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    total = sum(sum(v) for v in dur.values())
    out = [f"# {args.title}", ""]
    out += ["Commands (from the repository root, on one MI355X):", "", "```", *commands(args), "```", ""]
    if args.note:
        out += [args.note, ""]
    out += ["| kernel | calls | avg us | min us | max us | % time |", "|---|---:|---:|---:|---:|---:|"]
    for name, v in sorted(dur.items(), key=lambda kv: -sum(kv[1])):
        if sum(v) / total < 1e-4:
            continue
        out.append(f"| `{name[:100]}` ({short(name)}) | {len(v)} | {statistics.mean(v):.1f} | {min(v):.1f} | "
                   f"{max(v):.1f} | {100 * sum(v) / total:.2f} |")
    euler = [i for i, r in enumerate(rows) if "euler_kernel" in r["Kernel_Name"]]
    K = args.steps
    if len(euler) > K:
        seg = rows[euler[-K - 1] + 1: euler[-1] + 1]
        busy = sum(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in seg) / 1e6
        span = (int(seg[-1]["End_Timestamp"]) - int(seg[0]["Start_Timestamp"])) / 1e6
        inner = rows[euler[-K] + 1: euler[-1] + 1]
        inner_idle = ((int(inner[-1]["End_Timestamp"]) - int(rows[euler[-K]]["End_Timestamp"])) -
                      sum(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in inner)) / 1e6
        out += ["", f"## The last {K} Euler steps (the timed steps)", "",
                f"From the first kernel after the Euler update that precedes them to the last Euler update: "
                f"{len(seg)} dispatches, span {span:.2f} ms = {span / K:.2f} ms per step; device busy "
                f"{busy:.2f} ms; idle between kernels {span - busy:.3f} ms = **{(span - busy) / K:.3f} ms per "
                f"step**. Within one denoise call (the last {K - 1} steps, from the end of the first of the "
                f"{K} Euler updates): {inner_idle:.3f} ms idle = **{inner_idle / (K - 1):.3f} ms per step**; the "
                f"rest is the host's work between two calls (the previous call's result copy and synchronisation, "
                f"the next call's set-up).", "",
                "Stage time per step (dispatch durations, reductions and combines with their stage):", "",
                "| stage | dispatches / step | ms / step | avg us / launch (with its reductions) |", "|---|---:|---:|---:|"]
        stage_ms = defaultdict(float)
        stage_n = defaultdict(int)
        launches = defaultdict(int)
        prev = None
        for r in seg:
            st, main_kernel = stage_of(r["Kernel_Name"], prev)
            prev = st
            key = st or "other (" + short(r["Kernel_Name"]) + ")"
            stage_ms[key] += (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e6
            stage_n[key] += 1
            launches[key] += main_kernel or not st
        for key, ms in sorted(stage_ms.items(), key=lambda kv: -kv[1]):
            out.append(f"| {key} | {stage_n[key] / K:g} | {ms / K:.3f} | {1e3 * ms / launches[key]:.1f} |")
        gaps = defaultdict(list)
        for a, b in zip(seg, seg[1:]):
            gaps[(short(a["Kernel_Name"]), short(b["Kernel_Name"]))].append(
                (int(b["Start_Timestamp"]) - int(a["End_Timestamp"])) / 1e3)
        out += ["", "Largest idle totals between consecutive kernels:", "",
                "| after | before | count | avg us | max us | total us / step |", "|---|---|---:|---:|---:|---:|"]
        for (a, b), v in sorted(gaps.items(), key=lambda kv: -sum(kv[1]))[:args.gaps]:
            out.append(f"| {a} | {b} | {len(v)} | {statistics.mean(v):.2f} | {max(v):.1f} | {sum(v) / K:.1f} |")
    if args.bench_log:
        out += bench_classes(args.bench_log)
    emit(args, out)


def counter_rows(directory, counter):
    rows = [r for r in read_csv(directory, "_counter_collection.csv") if r["Counter_Name"] == counter]
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    return rows


def traffic(args):
    fetch = counter_rows(args.fetch_dir, "FETCH_SIZE")
    write = counter_rows(args.write_dir, "WRITE_SIZE")
    copy_bytes = args.copy_mib * 2**20

    def calibration(rows, name):
        """The first args.copies dispatches (the copies bench.py makes before any other
        kernel) and the rest."""
        n = args.copies
        if len(rows) <= n or any("convert_kernel" not in r["Kernel_Name"] for r in rows[:n]):
            sys.exit(f"the {name} run does not start with {n} calibration copies")
        mean = statistics.mean(float(r["Counter_Value"]) for r in rows[:n])
        return mean, copy_bytes / (mean * 1024), rows[n:]

    f_cal, f_scale, seq_f = calibration(fetch, "FETCH_SIZE")
    w_cal, w_scale, seq_w = calibration(write, "WRITE_SIZE")
    if [r["Kernel_Name"] for r in seq_f] != [r["Kernel_Name"] for r in seq_w]:
        sys.exit("the two runs dispatched different kernel sequences")
    per_kernel = defaultdict(lambda: [0, 0.0, 0.0])
    stage_bytes = defaultdict(float)
    stage_launches = defaultdict(int)
    prev = None
    for rf, rw in zip(seq_f, seq_w):
        name = rf["Kernel_Name"]
        fb = float(rf["Counter_Value"]) * 1024 * f_scale
        wb = float(rw["Counter_Value"]) * 1024 * w_scale
        k = per_kernel[name]
        k[0] += 1
        k[1] += fb
        k[2] += wb
        st, main_kernel = stage_of(name, prev)
        prev = st
        if st:
            stage_bytes[st] += fb + wb
            stage_launches[st] += main_kernel
    out = [f"# {args.title}", "", "Two counter runs (one counter each), from the repository root on one MI355X:", "",
           "```", *commands(args), "```", "",
           f"Calibration: the plain FP32 copy kernel (`convert_kernel`, {args.copy_mib} MiB read + {args.copy_mib} MiB "
           f"written per dispatch) reads FETCH_SIZE = {f_cal:.0f} KiB and WRITE_SIZE = {w_cal:.0f} KiB, so bytes = "
           f"FETCH_SIZE x 1024 x {f_scale:.3f} and WRITE_SIZE x 1024 x {w_scale:.3f}.", "",
           "| kernel | dispatches | read MB / dispatch | written MB / dispatch |", "|---|---:|---:|---:|"]
    for name, (n, fb, wb) in per_kernel.items():
        out.append(f"| `{name[:100]}` ({short(name)}) | {n} | {fb / n / 1e6:.1f} | {wb / n / 1e6:.1f} |")
    per_launch = {st: stage_bytes[st] / stage_launches[st] for st in stage_bytes if stage_launches[st]}
    out += ["", "Per launch of each block stage (its main kernel plus the split-K reduction, SDPA combine or "
            "split-tail pass that follows it):", "", "| stage | launches | HBM MB / launch |", "|---|---:|---:|"]
    for st, b in per_launch.items():
        out.append(f"| {st} | {stage_launches[st]} | {b / 1e6:.1f} |")
    record = {"kernel_sources_sha256": args.sources_sha256,
              "bytes_per_launch": {st: round(b) for st, b in per_launch.items()}}
    out += ["", "```json traffic", json.dumps(record, indent=1), "```"]
    emit(args, out)


def mfma(args):
    rows = read_csv(args.dir, "_counter_collection.csv")
    per = defaultdict(lambda: defaultdict(list))
    dur = defaultdict(dict)
    for r in rows:
        per[r["Kernel_Name"]][r["Counter_Name"]].append(float(r["Counter_Value"]))
        dur[r["Kernel_Name"]][r["Dispatch_Id"]] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    out = [f"# {args.title}", "", "One counter run, from the repository root on one MI355X:", "", "```",
           *commands(args), "```", "",
           "Per dispatch means. GRBM_GUI_ACTIVE is summed over the 8 XCDs, so the clock the kernel ran at is "
           "GUI / 8 / duration (dispatch timestamps of this run, kernels serialised by the profiler). "
           "SQ_VALU_MFMA_BUSY_CYCLES is summed over the 1024 SIMDs, so MFMA busy = MFMA_BUSY / (1024 x GUI / 8): "
           "the fraction of SIMD cycles the matrix cores work, at the clock the chip actually ran.", "",
           "| kernel | dispatches | us | clock GHz | MFMA busy | VALU instr / MFMA | LDS instr / MFMA |",
           "|---|---:|---:|---:|---:|---:|---:|"]
    for name, c in per.items():
        m = {k: statistics.mean(v) for k, v in c.items()}
        us = statistics.mean(dur[name].values())
        gui = m.get("GRBM_GUI_ACTIVE", 0) / 8
        busy = m.get("SQ_VALU_MFMA_BUSY_CYCLES", 0) / (1024 * gui) if gui else float("nan")
        n_mfma = m.get("SQ_INSTS_MFMA", 0)
        ratio = (lambda k: f"{m[k] / n_mfma:.2f}" if n_mfma and k in m else "-")
        out.append(f"| `{name[:90]}` ({short(name)}) | {len(dur[name])} | {us:.1f} | {gui / us / 1e3:.2f} | "
                   f"{busy:.3f} | {ratio('SQ_INSTS_VALU')} | {ratio('SQ_INSTS_LDS')} |")
    emit(args, out)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = ap.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("trace")
    t.add_argument("dir")
    t.add_argument("--steps", type=int, default=8)
    t.add_argument("--gaps", type=int, default=12)
    t.add_argument("--title", default="Kernel trace")
    t.add_argument("--command", action="append", default=[])
    t.add_argument("--note", default="")
    t.add_argument("--bench-log", default="", help="bench.py output of the traced run: its HIP-event class table")
    f = sub.add_parser("traffic")
    f.add_argument("fetch_dir")
    f.add_argument("write_dir")
    f.add_argument("--copy-mib", type=int, default=512)
    f.add_argument("--copies", type=int, default=3)
    f.add_argument("--sources-sha256", required=True)
    f.add_argument("--title", default="HBM traffic per dispatch (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE)")
    f.add_argument("--command", action="append", default=[])
    m = sub.add_parser("mfma")
    m.add_argument("dir")
    m.add_argument("--title", default="MFMA and VALU counters")
    m.add_argument("--command", action="append", default=[])
    for p in (t, f, m):
        p.add_argument("--output", default="", help="write the summary here instead of stdout")
    args = ap.parse_args(argv)
    {"trace": trace, "traffic": traffic, "mfma": mfma}[args.cmd](args)


if __name__ == "__main__":
    main()
