"""Benchmark of the MI355X paged GQA decode path (one GPU).

Headline workload (the "Llama-3-8B shape"): batch
64, 32 q / 8 kv heads, head_dim 128, page 16, every sequence 4096 tokens, fp16
paged KV in a fully permuted 16,384-block pool, split-KV on. One "step" is one
decode call (`pagedattn.paged_decode_triton`) over the whole batch, inputs
resident in HBM. K/V are rotated over `--copies` identical pool copies so the
256 MB MALL cannot serve a call from the previous one.

Prints ONE JSON line: value = algorithmic HBM GB/s of a whole decode call
(K+V+q+out+block-table bytes / call time), plus µs/call, a roofline object for
the dominant decode kernel (HIP-event timed, launched alone) and a CPU
baseline (the torch fp32 oracle on the same workload). Without --config the
line also carries `configs`: the other BASELINE.json configs (C1, C3, C4,
C5), each measured the same way in the same process (whole call, decode
kernel alone, merge alone, HIP-graph whole call, sampled-row parity, bit
stability, traffic ratio), with C1's CPU baseline on its full 24-row call.

Timing: `us_per_call` (and `value`) is the mean over the --steps timed calls,
one HIP event pair around them, with one more untimed call queued just before
the start event (no sync between), so the pair times steady-state calls rather
than the slow first call after the synchronize; the same loop is run LOOP_REPEATS more times
for `us_per_call_median` and `us_per_call_range` (median and extremes of the
loops' means). The decode kernel alone is timed eagerly and as a replayed
HIP graph; `kernel_us` is the graph figure for launches that take no host
launch tables (the captured code path is the same, and the host's launch rate
cannot set it: C1), else the eager one (a captured flat launch scans
seq_lens instead of using the host tables). Merge and whole-call graph
figures are medians of GRAPH_REPLAYS replays after a clock settle; a
captured flat merge scans seq_lens too.

    python bench.py [--gpus 1] [--steps 100] [--warmup 10] [--config c2]
"""

from __future__ import annotations

import argparse
import ctypes
import dataclasses
import hashlib
import json
import math
import os
import pathlib
import statistics
import sys
import time
import types

ROOT = pathlib.Path(__file__).resolve().parent
PKG = ROOT / "paged-decode-attention_amd"
for _p in (str(PKG), str(ROOT)):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, published


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


@dataclasses.dataclass
class Workload:
    name: str
    shape_name: str
    batch: int
    lens: list
    kv_dtype: str
    scale_fp32: bool
    pool_blocks: int
    seed: int
    description: str


def make_workload(cfg: str) -> Workload:
    """The BASELINE.json configs, generated deterministically."""
    import torch

    from pagedattn import LLAMA3_8B, LLAMA3_70B, QWEN25_05B

    if cfg == "c1":
        g = torch.Generator().manual_seed(0)
        lens = torch.randint(32, 193, (24,), generator=g).tolist()
        return Workload("c1", QWEN25_05B.name, 24, lens, "fp16", False, 512, 0,
                        "Qwen2.5-0.5B shape 14q/2kv d64, B=24, T~U[32,192], fp16, 512-block pool")
    if cfg == "c2":
        return Workload("c2", LLAMA3_8B.name, 64, [4096] * 64, "fp16", False, 64 * 256, 1,
                        "Llama-3-8B shape 32q/8kv d128, B=64, T=4096, fp16, page 16")
    if cfg == "c3":
        g = torch.Generator().manual_seed(2)
        u = torch.rand(64, generator=g, dtype=torch.float64)
        lens = torch.exp(math.log(128) + u * (math.log(8192) - math.log(128))).round().long().tolist()
        nb = sum(-(-t // 16) for t in lens)
        return Workload("c3", LLAMA3_8B.name, 64, lens, "fp8_e5m2", False, nb, 2,
                        "Llama-3-8B shape, fp8_e5m2 KV, B=64, T log-uniform 128..8192")
    if cfg == "c4":
        return Workload("c4", LLAMA3_70B.name, 32, [16384] * 32, "int8", True, 32 * 1024, 3,
                        "64q/8kv d128 (g8), B=32, T=16384, int8 KV + fp32 per-(token,head) scales")
    if cfg == "c5":
        return Workload("c5", LLAMA3_8B.name, 4, [131072] * 4, "fp16", False, 40_000, 4,
                        "32q/8kv d128, B=4, T=131072, fp16, 40k-block shuffled pool")
    raise SystemExit(f"unknown config {cfg}")


def shape_of(name: str):
    from pagedattn import LLAMA3_8B, LLAMA3_70B, QWEN25_05B

    return {s.name: s for s in (LLAMA3_8B, LLAMA3_70B, QWEN25_05B)}[name]


def subset_cache(cache, rows):
    """CPU copy of batch rows `rows` of a device cache, blocks renumbered."""
    import torch

    bt = cache.block_table.cpu()
    lens = cache.seq_lens.cpu()
    bs = cache.block_size
    ids, new_bt = [], []
    for r in rows:
        n = -(-int(lens[r]) // bs)
        base = sum(len(x) for x in ids)
        ids.append(bt[r, :n].long())
        row = torch.zeros(bt.shape[1], dtype=torch.int32)
        row[:n] = torch.arange(base, base + n, dtype=torch.int32)
        new_bt.append(row)
    dev_ids = torch.cat(ids).to(cache.k_cache.device)
    pick = lambda t: None if t is None else t.index_select(0, dev_ids).cpu()
    return types.SimpleNamespace(
        shape=cache.shape, block_size=bs, kv_dtype=cache.kv_dtype,
        k_cache=pick(cache.k_cache), v_cache=pick(cache.v_cache),
        k_scale=pick(cache.k_scale), v_scale=pick(cache.v_scale),
        block_table=torch.stack(new_bt), seq_lens=lens[list(rows)].clone(),
    )


def cpu_baseline(q, cache, budget_s: float, max_rows: int | None = None) -> dict:
    """The torch fp32 oracle (a port of pagedattn/reference.py:28-49) timed on
    the host on a bounded sample of the workload's sequences: as many as
    three runs fit in `budget_s` (all of them when the whole call fits)."""
    import torch

    from oracle import reference as oracle

    threads = min(16, os.cpu_count() or 1)
    torch.set_num_threads(threads)
    b = cache.batch
    probe = subset_cache(cache, [0])
    t0 = time.perf_counter()
    oracle.reference_decode(q[:1].cpu(), probe)
    per_seq = max(time.perf_counter() - t0, 1e-4)
    # as many sequences as three runs fit in the budget, then as many runs
    # (3 to 15) as the budget holds, for a stable median
    n = int(max(1, min(b, max_rows or b, budget_s / (3 * per_seq))))
    runs = int(max(3, min(15, budget_s / (n * per_seq))))
    rows = list(range(n))
    sub = subset_cache(cache, rows)
    qs = q[:n].cpu()
    oracle.reference_decode(qs, sub)  # warm-up
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        oracle.reference_decode(qs, sub)
        times.append(time.perf_counter() - t0)
    med = sorted(times)[len(times) // 2]
    sub_bytes = _algorithmic_bytes(sub)
    whole = "the whole call" if n == b else f"the first {n} of {b} sequences"
    return {
        "value": round(sub_bytes / med / 1e9, 4),
        "unit": "GB/s",
        "cores": threads,
        "cpu_count": os.cpu_count(),
        "torch_threads": torch.get_num_threads(),
        "kind": "port",
        "us_per_call": round(med * b / n * 1e6, 1),
        "sample": f"oracle.reference_decode (torch fp32 CPU, gather + per-head einsum) on {whole}, "
                  f"median of {runs} runs after one warm-up: {med * 1e3:.2f} ms for "
                  f"{sub_bytes / 1e6:.2f} MB algorithmic; {torch.get_num_threads()} torch threads "
                  f"of {os.cpu_count()} host CPUs",
    }


CLOCK_SETTLE_S = 0.25


def settle(step, seconds: float = CLOCK_SETTLE_S) -> None:
    """Run `step(i)` untimed for `seconds` of wall time (synchronising every
    16 calls so the host does not queue far ahead of the GPU)."""
    import torch

    t_end = time.perf_counter() + seconds
    i = 0
    while time.perf_counter() < t_end:
        step(i)
        i += 1
        if i % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def _algo_bytes(lens, shape, elem: int, scale_bytes: int, block_size: int) -> int:
    """K/V (+ int8 scales) inside the sequences + q + out (fp16) + used
    block-table entries."""
    n_tok = sum(int(t) for t in lens)
    kv = 2 * n_tok * shape.num_kv_heads * shape.head_dim * elem
    kv += 2 * n_tok * shape.num_kv_heads * scale_bytes
    pages = sum(-(-int(t) // block_size) for t in lens)
    return kv + 2 * len(lens) * shape.num_q_heads * shape.head_dim * 2 + 4 * pages


def _algorithmic_bytes(cache) -> int:
    scale = cache.k_scale.element_size() if cache.kv_dtype == "int8" else 0
    return _algo_bytes(cache.seq_lens.cpu().tolist(), cache.shape, cache.k_cache.element_size(), scale,
                       cache.block_size)


def _workload_algo_bytes(wl: "Workload") -> int:
    elem = {"fp16": 2, "bf16": 2, "fp8_e5m2": 1, "int8": 1}[wl.kv_dtype]
    scale = (4 if wl.scale_fp32 else 2) if wl.kv_dtype == "int8" else 0
    return _algo_bytes(wl.lens, shape_of(wl.shape_name), elem, scale, 16)


def bench_write(args, wl, shape, cache, dev) -> int:
    """The KV-cache write (pa_cache_write) of --write-tokens fp16 K/V rows into
    random slots of the workload's pool, in the workload's KV dtype; checked
    bit-exact against the oracle on a sample first."""
    import torch

    from oracle import reference as oracle
    from pagedattn import reshape_and_cache

    n = min(args.write_tokens, cache.k_cache.shape[0] * cache.block_size)
    g = torch.Generator().manual_seed(7)
    h, d = shape.num_kv_heads, shape.head_dim
    key = torch.randn((n, h, d), generator=g, dtype=torch.float16).to(dev)
    value = torch.randn((n, h, d), generator=g, dtype=torch.float16).to(dev)
    slots = torch.randperm(cache.k_cache.shape[0] * cache.block_size, generator=g)[:n].to(dev)
    # parity on a 64-row sample
    sample = slots[:64].cpu()
    reshape_and_cache(key[:64], value[:64], cache, slots[:64])
    torch.cuda.synchronize()
    blk, off = sample // cache.block_size, sample % cache.block_size
    want_k, want_ks = oracle.quantize_kv(key[:64].cpu(), cache.kv_dtype,
                                         cache.k_scale.dtype if cache.k_scale is not None else torch.float16)
    got_k = cache.k_cache[blk.to(dev), off.to(dev)].cpu()
    raw = lambda t: t.view(torch.uint8) if t.element_size() == 1 else t
    exact = bool(torch.equal(raw(got_k), raw(want_k)))
    if want_ks is not None:
        exact = exact and bool(torch.equal(cache.k_scale[blk.to(dev), off.to(dev)].cpu(), want_ks))
    _log(f"write parity on 64 rows: bit-exact={exact}")
    if not exact:
        return 1
    settle(lambda i: reshape_and_cache(key, value, cache, slots))
    for _ in range(args.warmup):
        reshape_and_cache(key, value, cache, slots)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    _prime(lambda: reshape_and_cache(key, value, cache, slots))
    ev0.record()
    for _ in range(args.steps):
        reshape_and_cache(key, value, cache, slots)
    ev1.record()
    torch.cuda.synchronize()
    us = ev0.elapsed_time(ev1) / args.steps * 1e3
    elem = cache.k_cache.element_size()
    sbytes = 0 if cache.k_scale is None else cache.k_scale.element_size()
    algo = n * h * d * 2 * 2 + n * h * d * elem * 2 + n * 8 + n * h * sbytes * 2
    gbs = algo / (us * 1e-6) / 1e9
    print(json.dumps({
        "metric": "kv cache write GB/s", "value": round(gbs, 2), "unit": "GB/s",
        "us_per_call": round(us, 2), "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "higher_is_better": True, "dtype": cache.kv_dtype, "data": "synthetic",
        "config": {"workload": f"{wl.name} pool, {n} rows [{h}, {d}] fp16 -> {cache.kv_dtype}"},
        "algorithmic_bytes_per_call": algo, "parity_bit_exact": exact,
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "cache_write_kernel",
                     "kernel_us": round(us, 2)},
    }), flush=True)
    return 0




def kernel_source_hash() -> str:
    """Hash of the HIP sources (csrc/*.hip, *.h): traffic counters measured
    on other sources do not describe the kernels that run."""
    h = hashlib.sha256()
    for p in sorted((PKG / "csrc").iterdir()):
        if p.suffix in (".hip", ".h"):
            h.update(p.name.encode())
            h.update(p.read_bytes())
    return h.hexdigest()[:16]


def traffic_for(cfg: str, kernel_name: str) -> tuple[int | None, str]:
    """HBM bytes per decode launch from profiles/traffic.json (rocprofv3
    FETCH_SIZE / WRITE_SIZE runs, calibrated), with the reason when there is
    none: no entry, another kernel, or counters of other kernel sources."""
    tfile = ROOT / "profiles" / "traffic.json"
    try:
        entry = json.loads(tfile.read_text()).get(cfg)
    except (OSError, ValueError):
        return None, "profiles/traffic.json unreadable"
    if not entry:
        return None, f"no counters for {cfg}"
    if entry.get("kernel") != kernel_name:
        return None, f"counters are for {entry.get('kernel')}, not {kernel_name}"
    if entry.get("source_hash") != kernel_source_hash():
        return None, (f"counters were taken on kernel sources {entry.get('source_hash')}, "
                      f"these are {kernel_source_hash()}")
    return entry.get("hbm_bytes_per_launch"), entry.get("source", "")


CALIB_COPY_BYTES = 1 << 30  # the --calib-copy device copy


def _counter_rows(path: str, counter: str) -> list[tuple[str, float]]:
    """(kernel name, value in KiB) per dispatch of a rocprofv3 --pmc CSV."""
    import csv

    with open(path, newline="") as f:
        return [(r["Kernel_Name"], float(r["Counter_Value"])) for r in csv.DictReader(f)
                if r["Counter_Name"] == counter]


def record_traffic(cfg: str, fetch_csv: str, write_csv: str) -> int:
    """Turn two rocprofv3 counter runs of `bench.py --config cfg --calib-copy`
    (one with --pmc FETCH_SIZE, one with --pmc WRITE_SIZE) into HBM bytes per
    decode launch: each counter's mean over the decode kernel's dispatches,
    scaled by what the same counter reads for the 1 GiB calibration copy
    (the largest __amd_rocclr_copyBuffer dispatches). Writes the entry of
    profiles/traffic.json, keyed to the current kernel sources, and the
    summary profiles/paged_decode_<cfg>_hbm_counters.md. Runs on the CPU."""
    import statistics

    wl = make_workload(cfg)
    algo = _workload_algo_bytes(wl)
    kib = CALIB_COPY_BYTES / 1024
    out = {}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        rows = _counter_rows(path, counter)
        copies = [v for n, v in rows if "copyBuffer" in n]
        big = [v for v in copies if v > 0.25 * kib] if counter == "FETCH_SIZE" else \
              [v for v in copies if v > 0.5 * kib]
        if not big:
            raise SystemExit(f"{path}: no calibration copy (run bench.py with --calib-copy)")
        factor = kib / statistics.median(big)
        per = {}
        for name, v in rows:
            for k in ("paged_decode_flat_kernel", "paged_decode_kernel", "split_reduce_kernel",
                      "flat_merge_table_kernel"):
                if k + "<" in name:
                    per.setdefault(k, []).append(v)
        out[counter] = (factor, {k: (statistics.fmean(v), len(v)) for k, v in per.items()},
                        statistics.median(big))
    (ff, fetch, fcal), (wf, write, wcal) = out["FETCH_SIZE"], out["WRITE_SIZE"]
    kernel = "paged_decode_flat_kernel" if "paged_decode_flat_kernel" in fetch else "paged_decode_kernel"
    if kernel not in fetch or kernel not in write:
        raise SystemExit(f"no {kernel} dispatches in the counter files")
    hbm = {k: fetch[k][0] * 1024 * ff + write[k][0] * 1024 * wf for k in fetch if k in write}
    tfile = ROOT / "profiles" / "traffic.json"
    data = json.loads(tfile.read_text()) if tfile.exists() else {}
    summary = f"profiles/paged_decode_{cfg}_hbm_counters.md"
    data[cfg] = {"kernel": kernel, "hbm_bytes_per_launch": round(hbm[kernel]),
                 "fetch_factor": round(ff, 4), "write_factor": round(wf, 4),
                 "source_hash": kernel_source_hash(), "source": summary}
    tfile.write_text(json.dumps(data, indent=1, sort_keys=True) + "\n")
    lines = [
        f"# rocprofv3 HBM counters — paged decode, {cfg}",
        "",
        f"Workload: {wl.name}: {wl.description}. Kernel sources: `{kernel_source_hash()}` "
        "(sha256 prefix of csrc/*.hip, *.h, as `bench.py` computes it).",
        "",
        "Commands (two runs; FETCH_SIZE and WRITE_SIZE each in a pass of its own), then the summary",
        "on the CPU:",
        "",
        "```",
        "cd /root/repo && export TMPDIR=/tmp",
        f"rocprofv3 --pmc FETCH_SIZE -d gpurun_out/pmc_FETCH_SIZE_{cfg} -o {cfg} --output-format csv -- "
        f"python3 bench.py --config {cfg} --steps 10 --warmup 2 --no-cpu --calib-copy",
        f"rocprofv3 --pmc WRITE_SIZE -d gpurun_out/pmc_WRITE_SIZE_{cfg} -o {cfg} --output-format csv -- "
        f"python3 bench.py --config {cfg} --steps 10 --warmup 2 --no-cpu --calib-copy",
        f"python3 bench.py --config {cfg} --record-traffic "
        f"gpurun_out/pmc_FETCH_SIZE_{cfg}/{cfg}_counter_collection.csv "
        f"gpurun_out/pmc_WRITE_SIZE_{cfg}/{cfg}_counter_collection.csv",
        "```",
        "",
        f"Calibration: the 1 GiB device copy (`__amd_rocclr_copyBuffer`) reads FETCH_SIZE "
        f"{fcal:,.0f} KiB for {kib:,.0f} KiB read (factor {ff:.4f}) and WRITE_SIZE {wcal:,.0f} KiB "
        f"for {kib:,.0f} KiB written (factor {wf:.4f}).",
        "",
        "| kernel | dispatches | FETCH_SIZE KiB (mean) | WRITE_SIZE KiB (mean) | calibrated HBM bytes / launch |",
        "|---|---:|---:|---:|---:|",
    ]
    for k in sorted(hbm, key=lambda k: -hbm[k]):
        lines.append(f"| `{k}` | {fetch[k][1]} | {fetch[k][0]:,.1f} | {write[k][0]:,.1f} | {hbm[k]:,.0f} |")
    lines += ["", f"Algorithmic bytes per decode call: {algo:,}. Calibrated traffic of `{kernel}` / "
                  f"algorithmic = {hbm[kernel] / algo:.4f}.", ""]
    (ROOT / summary).write_text("\n".join(lines))
    _log(f"{cfg}: {kernel} {hbm[kernel]:,.0f} B/launch = {hbm[kernel] / algo:.4f} x algorithmic "
         f"(fetch x{ff:.3f}, write x{wf:.3f}); wrote {summary}")
    return 0


def record_trace(cfg: str, stats_csv: str, trace_csv: str, bench_out: str) -> int:
    """Summarise a `rocprofv3 --kernel-trace --stats` run of `bench.py
    --config cfg` into profiles/paged_decode_<cfg>_kernel_trace.md: the top
    kernels, the bench line the same run printed, and the decode kernel's
    rocprof durations over the bench's two kernel-alone loops (the eager one,
    its last --steps dispatches, and the replayed graph, its last
    GRAPH_CALLS x GRAPH_REPLAYS dispatches; the bench brackets both with
    phase-marker kernels) beside the bench's HIP-event figures. Runs on the
    CPU."""
    import csv
    import statistics

    wl = make_workload(cfg)
    line = next(l for l in reversed(pathlib.Path(bench_out).read_text().splitlines()) if l.startswith("{"))
    bench = json.loads(line)
    steps = int(bench["steps"])
    with open(stats_csv, newline="") as f:
        stats = list(csv.DictReader(f))
    with open(trace_csv, newline="") as f:
        trace = [(int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]) for r in csv.DictReader(f)]
    trace.sort()
    kernel = bench["roofline"]["kernel"]
    marks = [i for i, (_, _, name) in enumerate(trace) if "spin_kernel" in name]
    if len(marks) < 3:
        raise SystemExit(f"{trace_csv}: {len(marks)} phase markers (spin_kernel), need 3")
    between = lambda a, b: [(t1 - t0) / 1e3 for t0, t1, name in trace[a + 1:b] if kernel + "<" in name]
    alone = between(marks[0], marks[1])[-steps:]
    graph = between(marks[1], marks[2])[-GRAPH_CALLS * GRAPH_REPLAYS:]
    short = lambda n: n.replace("(anonymous namespace)::", "").split("(")[0].replace("void ", "")[:90]
    cmd = (f"cd /root/repo && export TMPDIR=/tmp && rocprofv3 --kernel-trace --stats -d gpurun_out/trace_{cfg} "
           f"-o {cfg} --output-format csv -- python3 bench.py --config {cfg} --steps {steps} "
           f"--warmup {bench['warmup']} --no-cpu")
    lines = [
        f"# rocprofv3 kernel trace — paged decode, {cfg} ({wl.name}: {wl.description})",
        "",
        f"Kernel sources: `{kernel_source_hash()}`. Command (from the repo root, on one MI355X), then",
        "the summary on the CPU:",
        "",
        "```",
        cmd + f" > gpurun_out/trace_{cfg}.out",
        f"python3 bench.py --config {cfg} --record-trace gpurun_out/trace_{cfg}/{cfg}_kernel_stats.csv "
        f"gpurun_out/trace_{cfg}/{cfg}_kernel_trace.csv gpurun_out/trace_{cfg}.out",
        "```",
        "",
        f"Kernel stats (`{cfg}_kernel_stats.csv`, top entries; durations in µs):",
        "",
        "| kernel | calls | avg µs | min µs | max µs | % time |",
        "|---|---:|---:|---:|---:|---:|",
    ]
    for r in stats[:6]:
        lines.append(f"| `{short(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                     f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} | {float(r['Percentage']):.1f} |")
    avg, gavg = statistics.fmean(alone), statistics.fmean(graph)
    roof = bench["roofline"]
    lines += [
        "",
        f"Agreement, decode kernel `{kernel}` alone: the bench's eager loop (HIP events over {steps} "
        f"launches) = {roof['kernel_eager_us']:.2f} µs, the same {len(alone)} dispatches in rocprof's trace "
        f"average {avg:.2f} µs (median {statistics.median(alone):.2f}, min {min(alone):.2f}, max "
        f"{max(alone):.2f}); the bench's replayed graph = {roof['kernel_graph_us']:.2f} µs, its last "
        f"{len(graph)} dispatches average {gavg:.2f} µs (median {statistics.median(graph):.2f}). The bench "
        f"line's roofline uses kernel_us = {roof['kernel_us']:.2f} µs"
        + (" (the eager loop: the launch takes host launch tables, which a captured launch does not)."
           if roof["kernel_us"] == roof["kernel_eager_us"] else
           " (the replayed graph: the eager loop's launches wait for the host at this size).")
        + (" The eager loop is host-bound: each launch waits for the Python call that makes it, "
           "more so under the tracer, so its HIP-event figure exceeds the kernel's own time."
           if roof["kernel_eager_us"] > 1.2 * avg else ""),
        "",
        "The bench line printed by the same run:",
        "",
        "```",
        line,
        "```",
        "",
    ]
    out = ROOT / "profiles" / f"paged_decode_{cfg}_kernel_trace.md"
    out.write_text("\n".join(lines))
    _log(f"{cfg}: bench kernel {roof['kernel_eager_us']:.2f} / {roof['kernel_graph_us']:.2f} us (eager / graph), "
         f"rocprof {avg:.2f} / {gavg:.2f} us; wrote {out.name}")
    return 0


SQ_COUNTERS = ("SQ_WAVES", "SQ_INSTS_VALU", "SQ_INSTS_SALU", "SQ_INSTS_VMEM_RD", "SQ_INSTS_LDS",
               "SQ_WAVE_CYCLES", "SQ_BUSY_CYCLES", "SQ_WAIT_INST_ANY")


def record_sq(paths: list[str]) -> int:
    """Summarise rocprofv3 --pmc runs of the SQ_COUNTERS (one pass of eight,
    `bench.py --config cN`, files named `cN_counter_collection.csv`) into
    profiles/paged_decode_sq_instruction_counts.md: instructions per 32-token
    tile of one kv head for the flat decode kernel. Tiles per launch come
    from the workload (sum of ceil(T / 32) over the batch, times kv heads and
    head tiles). Runs on the CPU."""
    import csv
    import statistics

    rows_out = []
    for path in paths:
        cfg = pathlib.Path(path).name.split("_")[0]
        wl = make_workload(cfg)
        shape = shape_of(wl.shape_name)
        units = shape.num_kv_heads * -(-shape.gqa_group // 16)
        tiles = units * sum(-(-t // 32) for t in wl.lens)
        per = {}
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                if "paged_decode_flat_kernel<" in r["Kernel_Name"]:
                    per.setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
        if not per:
            raise SystemExit(f"{path}: no paged_decode_flat_kernel dispatches")
        m = {k: statistics.median(v) for k, v in per.items()}
        rows_out.append((cfg, wl, tiles, m))
    lines = [
        "# rocprofv3 SQ instruction counters — flat decode kernel",
        "",
        f"Kernel sources: `{kernel_source_hash()}`. Commands (from the repo root, on one MI355X; one pass",
        "of eight SQ counters per config), then the summary on the CPU:",
        "",
        "```",
        "cd /root/repo && export TMPDIR=/tmp",
        f"rocprofv3 --pmc {' '.join(SQ_COUNTERS)} -d gpurun_out/sq_cN -o cN --output-format csv -- "
        "python3 bench.py --config cN --steps 10 --warmup 2 --no-cpu",
        "python3 bench.py --record-sq " + " ".join(f"gpurun_out/sq_{c}/{c}_counter_collection.csv"
                                                  for c, _, _, _ in rows_out),
        "```",
        "",
        "Each counter is summed over the dispatch's dimensions, the median taken over the",
        "`paged_decode_flat_kernel` dispatches and divided by the tiles one launch computes (32",
        "tokens of one kv head each; MFMAs per tile: 8 for Q K^T and 8 for P V at head_dim 128).",
        "",
        "| config | waves | tiles / launch | VALU / tile | SALU / tile | LDS / tile | VMEM rd / tile | "
        "busy / wave cycles |",
        "|---|---:|---:|---:|---:|---:|---:|---:|",
    ]
    for cfg, wl, tiles, m in rows_out:
        g = lambda k: m.get(k, float("nan"))
        lines.append(f"| {cfg} ({wl.kv_dtype}) | {g('SQ_WAVES'):,.0f} | {tiles:,} | {g('SQ_INSTS_VALU') / tiles:.0f} | "
                     f"{g('SQ_INSTS_SALU') / tiles:.0f} | {g('SQ_INSTS_LDS') / tiles:.1f} | "
                     f"{g('SQ_INSTS_VMEM_RD') / tiles:.1f} | {g('SQ_BUSY_CYCLES'):,.0f} / {g('SQ_WAVE_CYCLES'):,.0f} |")
    lines.append("")
    out = ROOT / "profiles" / "paged_decode_sq_instruction_counts.md"
    out.write_text("\n".join(lines))
    _log(f"wrote {out.name}")
    return 0


GRAPH_CALLS = 20   # calls captured in one HIP graph
GRAPH_REPLAYS = 9  # replays timed one by one (the median is reported)


def _graph_us(fn, calls: int = GRAPH_CALLS, reps: int = GRAPH_REPLAYS) -> float:
    """µs per call of `fn(i)` for i < calls captured in one HIP graph: the
    graph is replayed untimed for CLOCK_SETTLE_S (the capture leaves the GPU
    idle), then `reps` replays are timed one by one with HIP events and the
    median replay is divided by `calls` (no host launch cost in the timed
    region)."""
    import statistics

    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn(0)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(calls):
            fn(i)
    settle(lambda i: graph.replay())
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(2 * reps)]
    _prime(graph.replay)
    for r in range(reps):
        evs[2 * r].record()
        graph.replay()
        evs[2 * r + 1].record()
    torch.cuda.synchronize()
    us = statistics.median(evs[2 * r].elapsed_time(evs[2 * r + 1]) for r in range(reps)) / calls * 1e3
    del graph
    return us


LOOP_REPEATS = 6  # extra timed loops of --steps calls, for the median and range


def _prime(fn) -> None:
    """One untimed call of the timed work, queued (no sync) right before a
    timed loop's start event. The loops follow a synchronize, and the first
    call after the GPU idles, even briefly, runs slow while the clocks come
    back: per-call events showed C2's first call at 175-240 us against ~163
    (C3: up to 88 against ~42), plus the host's first submission to an idle
    GPU. Queued ahead, that call absorbs both, and the event pair times K
    calls in steady state, as a serving loop runs them."""
    fn()


def _phase_marker() -> None:
    """A tiny kernel (torch's spin kernel) outside every timed region: in a
    rocprofv3 kernel trace the marker dispatches bracket the kernel-alone
    loops (eager, then the replayed graph), which `--record-trace` reads."""
    import torch

    torch.cuda._sleep(100)
    torch.cuda.synchronize()


def _loop_us(step, n: int, repeats: int) -> list[float]:
    """µs per call of `repeats` loops of `n` back-to-back calls of `step(i)`,
    each loop bracketed by one pair of HIP events on the current stream."""
    import torch

    evs = [torch.cuda.Event(enable_timing=True) for _ in range(2 * repeats)]
    _prime(lambda: step(0))
    for r in range(repeats):
        evs[2 * r].record()
        for i in range(n):
            step(i)
        evs[2 * r + 1].record()
    torch.cuda.synchronize()
    return [evs[2 * r].elapsed_time(evs[2 * r + 1]) * 1e3 / n for r in range(repeats)]


def measure(cfg: str, args, dev, cpu: bool) -> dict:
    """Time one BASELINE config on the GPU and check it. Returns the numbers
    and, under "_keep", the inputs (for the headline's CPU baseline)."""
    import torch

    from oracle import reference as oracle
    from pagedattn import allocate, flat_waves_per_simd, plan_launch, plan_num_splits
    from pagedattn.hip_decode import (_WS, _cu_count, decode_partials, flat_merge, paged_decode_hip,
                                      split_reduce)

    wl = make_workload(cfg)
    shape = shape_of(wl.shape_name)
    used = sum(-(-t // 16) for t in wl.lens)
    _log(f"config {wl.name}: {wl.description}; pool {wl.pool_blocks} blocks ({used} used)")
    t0 = time.perf_counter()
    sdt = torch.float32 if wl.scale_fp32 else torch.float16
    cache = allocate(shape, wl.batch, wl.lens, block_size=16, kv_dtype=wl.kv_dtype, device="cuda",
                     seed=wl.seed, slack_blocks=wl.pool_blocks - used, scale_dtype=sdt,
                     fill_device="cuda")
    g = torch.Generator().manual_seed(100 + wl.seed)
    q = torch.randn((wl.batch, shape.num_q_heads, shape.head_dim), dtype=torch.float16,
                    generator=g).to(dev)
    pool_bytes = 2 * cache.k_cache.numel() * cache.k_cache.element_size()
    copies = args.copies or max(1, math.ceil(512e6 / pool_bytes) + 1)
    caches = [cache]
    for _ in range(copies - 1):
        caches.append(dataclasses.replace(
            cache, k_cache=cache.k_cache.clone(), v_cache=cache.v_cache.clone(),
            k_scale=None if cache.k_scale is None else cache.k_scale.clone(),
            v_scale=None if cache.v_scale is None else cache.v_scale.clone()))
    torch.cuda.synchronize()
    _log(f"allocated {copies} pool copies of {pool_bytes / 2**30:.2f} GiB in {time.perf_counter() - t0:.1f} s")

    cus = _cu_count(dev)
    # the workload's lengths are known here, so the planner sees them all
    # unless --splits / --flat force a launch shape
    wps = flat_waves_per_simd(wl.kv_dtype, shape.head_dim, sdt)
    plan = plan_launch(wl.batch, 0, shape.num_kv_heads, shape.gqa_group, cus, wps,
                       kv_dtype=wl.kv_dtype, head_dim=shape.head_dim, seq_lens=wl.lens)
    splits, flat, cost = plan.num_splits, plan.flat_splits, plan.flat_seq_cost
    if args.flat is not None or args.splits:
        flat = int(args.flat or 0)
        splits = 1 if flat else (args.splits or
                                 plan_num_splits(wl.lens, shape.num_kv_heads, shape.gqa_group, cus)[0])
    if args.seq_cost is not None:
        cost = args.seq_cost
    cost = cost if flat else 0
    out = torch.empty_like(q)
    algo = _algorithmic_bytes(cache)
    msl = max(wl.lens)
    launch = (f"flat F={flat}" + (f" cost {cost}" if cost else "")) if flat else (
        "unsplit" if splits == 1 else f"split S={splits}")
    _log(f"{cus} CUs, {launch}, algorithmic bytes/call={algo}")

    # bit stability now; parity of sampled sequences against the CPU oracle
    # after the timed regions, so that seconds of CPU work do not leave the
    # GPU idle (and clocked down) right before them
    # the workload's lengths are known on the host, as a serving step's are
    host = None if (args.no_host_lens or not flat) else torch.tensor(wl.lens, dtype=torch.int32)
    if host is not None:
        launch += ", host lengths"
    step = lambda i: paged_decode_hip(q, caches[i % copies], out=out, num_splits=splits,
                                      max_seq_len=msl, flat_splits=flat, flat_seq_cost=cost,
                                      seq_lens_host=host)
    step(0)
    first = out.clone()
    step(0)
    torch.cuda.synchronize()
    bit_stable = bool(torch.equal(first, out))
    rows = sorted({0, wl.batch // 2, wl.batch - 1}) if wl.batch > 24 else list(range(wl.batch))
    got_rows = out[rows].float().cpu()

    if args.calib_copy:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # whole call (decode + merge when split), rotating pool copies. The GPU
    # comes out of idle at reduced clocks: at C4 the first ~100 calls after a
    # pause ran up to 30% slower. Untimed calls for CLOCK_SETTLE_S bring it
    # to the steady state of a serving loop before the warmup steps.
    settle(step)
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    _prime(lambda: step(0))
    ev0.record()
    t_wall = time.perf_counter()
    for i in range(args.steps):
        step(i)
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    ms_step = ev0.elapsed_time(ev1) / args.steps
    _log(f"whole call: {ms_step * 1e3:.1f} us/call (wall {wall / args.steps * 1e6:.1f} us/call)")
    # Spread: the same K-call loop repeated LOOP_REPEATS more times, each
    # timed by one event pair like the loop above; the median and range of
    # the loops' per-call means. (An event between every two calls would
    # time the events as well: it added 2-4 us per call.)
    loops = [ms_step * 1e3] + _loop_us(step, args.steps, LOOP_REPEATS)
    dist = {"median": statistics.median(loops), "min": min(loops), "max": max(loops), "loops": len(loops)}
    _log("loop means: median {median:.2f} us/call, min {min:.2f}, max {max:.2f} over {loops} loops".format(**dist))

    # the dominant kernel alone: the decode pass (partials when split)
    if flat:
        fo, fl = _WS.get_flat(wl.batch + flat, shape.num_q_heads, shape.head_dim, dev)
        run = lambda c: decode_partials(q, c, 1, part_out=fo, part_lse=fl, flat_splits=flat, out=out,
                                        flat_seq_cost=cost, seq_lens_host=host)
    elif splits > 1:
        part_out, part_lse = _WS.get(wl.batch, shape.num_q_heads, splits, shape.head_dim, dev)
        run = lambda c: decode_partials(q, c, splits, part_out=part_out, part_lse=part_lse,
                                         max_seq_len=msl)
    else:
        run = lambda c: paged_decode_hip(q, c, out=out, num_splits=1)
    _phase_marker()  # a kernel trace finds the kernel-alone loops between markers
    for i in range(args.warmup):
        run(caches[i % copies])
    torch.cuda.synchronize()
    _prime(lambda: run(caches[0]))
    ev0.record()
    for i in range(args.steps):
        run(caches[i % copies])
    ev1.record()
    torch.cuda.synchronize()
    kern_eager_us = ev0.elapsed_time(ev1) / args.steps * 1e3
    _log(f"decode kernel alone: {kern_eager_us:.1f} us/launch (eager)")
    _phase_marker()
    # The same launches replayed as a HIP graph, which the host's launch
    # rate cannot slow down (it does at C1, whose kernel takes a few us). A
    # captured flat launch takes no host launch tables (it scans seq_lens),
    # so for a launch with host tables the eager loop stays the kernel's
    # figure: it runs the product's code path, and at those sizes the host
    # keeps ahead of the GPU.
    kern_graph_us = _graph_us(lambda i: run(caches[i % copies]))
    _log(f"decode kernel alone: {kern_graph_us:.1f} us/launch (HIP graph)")
    _phase_marker()
    kern_us = kern_eager_us if host is not None else kern_graph_us

    # The merge pass alone. It is a few microseconds of GPU work, less than
    # one Python launch, so back-to-back eager launches would time the host:
    # the launches are captured in a HIP graph and the graph is replayed.
    reduce_us = None
    merge = None
    if flat:
        run(caches[0])  # the slots of one pass
        merge = lambda i: flat_merge(q, caches[0], flat, fo, fl, out, flat_seq_cost=cost, seq_lens_host=host)
    elif splits > 1:
        merge = lambda i: split_reduce(part_out, part_lse, out)
    if merge is not None:
        merge(0)
        torch.cuda.synchronize()
        eager = out.clone()
        reduce_us = _graph_us(merge)
        if not torch.equal(out, eager):
            raise RuntimeError("the merge graph's replay differs from the eager merge")
        _log(f"merge pass alone: {reduce_us:.2f} us/launch (graph of {GRAPH_CALLS} launches, median of "
             f"{GRAPH_REPLAYS} replays; captured, so a flat merge scans seq_lens)")
    # the whole call replayed as a graph: GPU time without the host's
    # launch cost (which dominates C1's eager call)
    graph_us = _graph_us(step)
    _log(f"whole call as a HIP graph: {graph_us:.1f} us/call")

    ref = oracle.reference_decode(q[rows].cpu(), subset_cache(cache, rows), out_dtype=torch.float32)
    max_abs = (got_rows - ref).abs().max().item()
    rel = max_abs / max(ref.abs().max().item(), 1e-6)
    _log(f"parity on rows {rows if len(rows) <= 3 else f'0..{wl.batch - 1}'}: max_abs_err={max_abs:.3e} "
         f"rel={rel:.2e}; bit_stable={bit_stable}")
    if not (max_abs < 2e-3) or not bit_stable:
        raise RuntimeError(f"{cfg}: PARITY FAILURE (max_abs {max_abs:.3e}, bit_stable {bit_stable})")

    kernel_name = "paged_decode_flat_kernel" if flat else "paged_decode_kernel"
    traffic, traffic_note = traffic_for(wl.name, kernel_name)
    res = {
        "wl": wl, "shape": shape, "splits": splits, "flat": flat, "seq_cost": cost, "launch": launch,
        "copies": copies,
        "us_per_call": ms_step * 1e3, "kernel_us": kern_us, "merge_us": reduce_us, "graph_us": graph_us,
        "kernel_eager_us": kern_eager_us, "kernel_graph_us": kern_graph_us, "dist": dist,
        "algo": algo, "kv_bytes": cache.bytes_read_per_decode_step(), "max_abs": max_abs, "rel": rel,
        "rows": rows, "bit_stable": bit_stable, "kernel_name": kernel_name, "traffic": traffic,
        "traffic_note": traffic_note,
    }
    if cpu:
        # the oracle on this config's inputs: the whole call when it fits
        # the budget (C1), a bounded sample otherwise
        res["cpu_baseline"] = cpu_baseline(q, cache, args.cpu_budget)
    del caches, cache, q, out
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return res


def _build_inputs(wl, shape, dev, copies_arg=None):
    """The workload's cache (GPU-filled, seeded), its rotated pool copies and q."""
    import torch

    from pagedattn import allocate

    used = sum(-(-t // 16) for t in wl.lens)
    sdt = torch.float32 if wl.scale_fp32 else torch.float16
    cache = allocate(shape, wl.batch, wl.lens, block_size=16, kv_dtype=wl.kv_dtype, device="cuda",
                     seed=wl.seed, slack_blocks=wl.pool_blocks - used, scale_dtype=sdt, fill_device="cuda")
    g = torch.Generator().manual_seed(100 + wl.seed)
    q = torch.randn((wl.batch, shape.num_q_heads, shape.head_dim), dtype=torch.float16, generator=g).to(dev)
    pool_bytes = 2 * cache.k_cache.numel() * cache.k_cache.element_size()
    copies = copies_arg or max(1, math.ceil(512e6 / pool_bytes) + 1)
    caches = [cache] + [dataclasses.replace(
        cache, k_cache=cache.k_cache.clone(), v_cache=cache.v_cache.clone(),
        k_scale=None if cache.k_scale is None else cache.k_scale.clone(),
        v_scale=None if cache.v_scale is None else cache.v_scale.clone()) for _ in range(copies - 1)]
    return cache, caches, q, sdt


def plan_check(args, dev) -> int:
    """Re-validate the launch planner on this GPU: for every BASELINE config,
    time the planner's launch against the other launch shapes (the flat
    split at the planner's range count, the per-sequence split, unsplit, and
    the flat split at half and twice the range count), each as an eager
    whole call (mean of --steps calls, rotating pool copies, flat launches
    with host lengths) and as a replayed HIP graph (median of replays). One
    JSON line per config; `margin_pct` is how much slower the fastest
    alternative is than the planner's choice (negative: an alternative won)."""
    import torch

    from pagedattn import flat_waves_per_simd, plan_launch, plan_num_splits, pick_num_splits
    from pagedattn.hip_decode import (RAGGED_FLAT_SEQ_COST, RAGGED_FLAT_SEQ_COST_KV, _cu_count,
                                      _nearly_uniform, flat_splits_for, paged_decode_hip)

    cfgs = [args.config] if args.config else ["c1", "c2", "c3", "c4", "c5"]
    for cfg in cfgs:
        wl = make_workload(cfg)
        shape = shape_of(wl.shape_name)
        cache, caches, q, sdt = _build_inputs(wl, shape, dev, args.copies)
        copies = len(caches)
        cus = _cu_count(dev)
        wps = flat_waves_per_simd(wl.kv_dtype, shape.head_dim, sdt)
        plan = plan_launch(wl.batch, 0, shape.num_kv_heads, shape.gqa_group, cus, wps, kv_dtype=wl.kv_dtype,
                           head_dim=shape.head_dim, seq_lens=wl.lens)
        flat = flat_splits_for(shape.num_kv_heads, shape.gqa_group, cus, wps, wl.kv_dtype)
        cost = 0 if _nearly_uniform(wl.lens) else RAGGED_FLAT_SEQ_COST_KV.get(wl.kv_dtype, RAGGED_FLAT_SEQ_COST)
        split = plan_num_splits(wl.lens, shape.num_kv_heads, shape.gqa_group, cus)[0]
        if split < 2:
            split = max(2, pick_num_splits(wl.batch, shape.num_kv_heads, max(wl.lens), cus))
        msl = max(wl.lens)
        variants = {
            "planned": plan.launch_kwargs(),
            f"flat F={flat}": {"flat_splits": flat, "flat_seq_cost": cost},
            f"flat F={max(1, flat // 2)}": {"flat_splits": max(1, flat // 2), "flat_seq_cost": cost},
            f"flat F={2 * flat}": {"flat_splits": 2 * flat, "flat_seq_cost": cost},
            f"split S={split}": {"num_splits": split, "max_seq_len": msl},
            "unsplit": {"num_splits": 1, "max_seq_len": msl},
        }
        host = torch.tensor(wl.lens, dtype=torch.int32)
        out = torch.empty_like(q)
        res = {}
        for name, kw in variants.items():
            kw = dict(kw)
            if kw.get("flat_splits"):
                kw["seq_lens_host"] = host
            step = lambda i, kw=kw: paged_decode_hip(q, caches[i % copies], out=out, **kw)
            settle(step)
            for i in range(args.warmup):
                step(i)
            eager = statistics.median(_loop_us(step, args.steps, 3))
            kw_graph = {k: v for k, v in kw.items() if k != "seq_lens_host"}
            graph = _graph_us(lambda i, kw=kw_graph: paged_decode_hip(q, caches[i % copies], out=out, **kw))
            res[name] = {"launch": {k: v for k, v in kw.items() if k != "seq_lens_host"},
                         "eager_us": round(eager, 2), "graph_us": round(graph, 2)}
            _log(f"{cfg} {name}: eager {eager:.2f} us, graph {graph:.2f} us")
        planned = res["planned"]
        same = [n for n, r in res.items() if n != "planned" and r["launch"] == planned["launch"]]
        alts = {n: r for n, r in res.items() if n != "planned" and n not in same}
        line = {"plan_check": cfg, "workload": wl.description, "cus": cus, "planned": planned,
                "planned_is": same, "alternatives": alts}
        for kind in ("eager_us", "graph_us"):
            best = min(alts.items(), key=lambda kv: kv[1][kind])
            line[f"best_alternative_{kind[:-3]}"] = best[0]
            line[f"margin_{kind[:-3]}_pct"] = round(100 * (best[1][kind] - planned[kind]) / planned[kind], 2)
        print(json.dumps(line), flush=True)
        del caches, cache, q, out
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return 0


def summary(r: dict) -> dict:
    """The compact per-config entry of the JSON line."""
    algo = r["algo"]
    wl = r["wl"]
    # BASELINE's 70% of 8 TB/s at this config's algorithmic bytes
    target_us = algo / (0.7 * HBM_PEAK_GBS * 1e9) * 1e6
    e = {
        "workload": wl.description,
        "launch": r["launch"],
        "us_per_call": round(r["us_per_call"], 2),
        "us_per_call_median": round(r["dist"]["median"], 2),
        "us_per_call_range": [round(r["dist"]["min"], 2), round(r["dist"]["max"], 2)],
        "graph_us_per_call": round(r["graph_us"], 2),
        "kernel_us": round(r["kernel_us"], 2),
        "kernel_eager_us": round(r["kernel_eager_us"], 2),
        "kernel_graph_us": round(r["kernel_graph_us"], 2),
        "merge_us": None if r["merge_us"] is None else round(r["merge_us"], 2),
        "algorithmic_bytes": algo,
        "gbs": round(algo / (r["us_per_call"] * 1e-6) / 1e9, 1),
        "pct_of_peak": round(100 * algo / (r["us_per_call"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 2),
        "kernel_frac": round(algo / (r["kernel_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "us_at_70pct": round(target_us, 1),
        "traffic_ratio": None if r["traffic"] is None else round(r["traffic"] / algo, 4),
        "parity_max_abs_err": float(f"{r['max_abs']:.3e}"),
        "parity_rows": len(r["rows"]),
        "bit_stable": r["bit_stable"],
    }
    if r["traffic"] is None:
        e["traffic_note"] = r["traffic_note"]
    if "cpu_baseline" in r:
        e["cpu_baseline"] = r["cpu_baseline"]
    return e


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default=None, choices=["c1", "c2", "c3", "c4", "c5"],
                    help="measure this config only (default: the headline c2, then c1, c3, c4, c5)")
    ap.add_argument("--splits", type=int, default=None, help="override the split count")
    ap.add_argument("--copies", type=int, default=None, help="pool copies rotated between calls")
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of CPU baseline work")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run a 1 GiB device copy (PMC calibration of FETCH/WRITE_SIZE)")
    ap.add_argument("--op", default="decode", choices=["decode", "write"],
                    help="decode (the headline) or write: the KV-cache write of --write-tokens rows")
    ap.add_argument("--write-tokens", type=int, default=65536)
    ap.add_argument("--flat", type=int, default=None,
                    help="flat (work-balanced) split with this many ranges per kv head; 0 = classic")
    ap.add_argument("--record-traffic", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"), default=None,
                    help="CPU only: fold two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) of "
                         "--config into profiles/traffic.json and its counter summary")
    ap.add_argument("--record-trace", nargs=3, metavar=("STATS_CSV", "TRACE_CSV", "BENCH_OUT"), default=None,
                    help="CPU only: summarise a rocprofv3 --kernel-trace --stats run of --config "
                         "into its profiles/ summary")
    ap.add_argument("--no-host-lens", action="store_true",
                    help="flat split: let the kernels scan seq_lens on the GPU instead of passing the "
                         "workload's lengths from the host (seq_lens_host)")
    ap.add_argument("--record-sq", nargs="+", metavar="CSV", default=None,
                    help="CPU only: summarise rocprofv3 SQ counter runs (cN_counter_collection.csv) "
                         "into profiles/paged_decode_sq_instruction_counts.md")
    ap.add_argument("--seq-cost", type=int, default=None,
                    help="override the flat split's per-sequence charge in tiles (flat_seq_cost)")
    ap.add_argument("--plan-check", action="store_true",
                    help="time the planner's launch against the other launch shapes on every config "
                         "(or --config), one JSON line per config")
    args = ap.parse_args()

    if args.record_traffic:
        if not args.config:
            raise SystemExit("--record-traffic needs --config")
        return record_traffic(args.config, *args.record_traffic)
    if args.record_sq:
        return record_sq(args.record_sq)
    if args.record_trace:
        if not args.config:
            raise SystemExit("--record-trace needs --config")
        return record_trace(args.config, *args.record_trace)

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the decode would shard over (batch, kv_head) with no exchange between "
              "GPUs). Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.plan_check:
        return plan_check(args, dev)

    if args.op == "write":
        from pagedattn import allocate

        wl = make_workload(args.config or "c2")
        shape = shape_of(wl.shape_name)
        used = sum(-(-t // 16) for t in wl.lens)
        cache = allocate(shape, wl.batch, wl.lens, block_size=16, kv_dtype=wl.kv_dtype, device="cuda",
                         seed=wl.seed, slack_blocks=wl.pool_blocks - used,
                         scale_dtype=torch.float32 if wl.scale_fp32 else torch.float16,
                         fill_device="cuda")
        return bench_write(args, wl, shape, cache, dev)

    head_cfg = args.config or "c2"
    try:
        h = measure(head_cfg, args, dev, cpu=not args.no_cpu)
        others = {}
        if args.config is None:
            for cfg in ("c1", "c3", "c4", "c5"):
                others[cfg] = summary(measure(cfg, args, dev, cpu=(cfg == "c1" and not args.no_cpu)))
    except RuntimeError as e:
        _log(str(e))
        return 1

    wl, shape = h["wl"], h["shape"]
    algo = h["algo"]
    ms_step = h["us_per_call"] / 1e3
    achieved_kernel = algo / (h["kernel_us"] * 1e-6) / 1e9
    value = algo / (ms_step * 1e-3) / 1e9
    result = {
        "metric": "decode attn µs/call + achieved HBM GB/s (% of peak), Llama-3-8B shape",
        "value": round(value, 2),
        "unit": "GB/s",
        "us_per_call": round(h["us_per_call"], 2),
        "us_per_call_median": round(h["dist"]["median"], 2),
        "us_per_call_range": [round(h["dist"]["min"], 2), round(h["dist"]["max"], 2)],
        "timed_loops": h["dist"]["loops"],
        "pct_of_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "clock_settle_s": CLOCK_SETTLE_S,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": wl.kv_dtype,
        "data": "synthetic (seeded N(0,1) fp16 K/V/q, permuted block pool)",
        "config": {
            "workload": f"{wl.name}: {wl.description}",
            "batch": wl.batch,
            "num_q_heads": shape.num_q_heads,
            "num_kv_heads": shape.num_kv_heads,
            "head_dim": shape.head_dim,
            "block_size": 16,
            "seq_len_max": max(wl.lens),
            "num_splits": h["splits"],
            "flat_splits": h["flat"],
            "flat_seq_cost": h["seq_cost"],
            "pool_copies_rotated": h["copies"],
            "parallelism": "single GPU",
        },
        "algorithmic_bytes_per_call": algo,
        "kv_bytes_per_call": h["kv_bytes"],
        "parity_max_abs_err": h["max_abs"],
        "bit_stable": h["bit_stable"],
        "split_reduce_us": None if h["merge_us"] is None else round(h["merge_us"], 3),
        "graph_us_per_call": round(h["graph_us"], 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved_kernel, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved_kernel / HBM_PEAK_GBS, 4),
            "traffic": h["traffic"],
            "kernel": h["kernel_name"],
            "kernel_us": round(h["kernel_us"], 2),
            "kernel_eager_us": round(h["kernel_eager_us"], 2),
            "kernel_graph_us": round(h["kernel_graph_us"], 2),
        },
        "cpu_baseline": h.get("cpu_baseline"),
    }
    if h["traffic"] is None:
        result["roofline"]["traffic_note"] = h["traffic_note"]
    if others:
        result["configs"] = others
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
