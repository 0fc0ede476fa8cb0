"""Attention-only decode loop: the part of a serving step this library owns.

The reference's integration/bench_vllm.py times a whole vLLM model. It keeps
a Result record (:43-61), checks the backend counters so that no number is
reported for a run its decode kernel never served (:162-170), and appends each
run to a JSON file (:297-307). That needs vLLM and a model checkpoint, neither
of which exists here. This loop keeps the record, the counters and the runs
file, for the attention part of each decode step. Each step grows every
sequence by one token on the device (the new token counts, as in vLLM's
seq_lens), then per layer:
  * writes the new token's K/V into the paged cache (`reshape_and_cache`, the
    step before the decode, integration/vllm_backend.py:117-122);
  * runs the decode with the launch the vLLM boundary would pick from the
    batch size and the longest length (`plan_launch` with no host-side
    lengths, so no device sync): the flat split, the unsplit kernel for a
    large batch of short sequences, or the classic split for a small batch
    (`--launch flat|unsplit` forces one).
With --graph the whole step is captured once as a HIP graph and replayed per
step, which is how a serving loop removes the per-launch host cost.

TPOT here is the attention share of time per output token: all layers' writes
and decodes of one step, timed with HIP events. There are no weights, MLPs,
sampling or prefill, and so no TTFT. A run ends with a self-check on the GPU:
the decode of the last step must agree with the other launch (unsplit for a
flat run, flat for an unsplit one) within 2e-3 plus one output ulp, and be
bit-stable.

usage (from the repository root):
  python paged-decode-attention_amd/integration/bench_decode_loop.py \\
      [--shape llama3-8b] [--layers 8] [--requests 64] [--prompt 4096] \\
      [--output-tokens 64] [--kv fp16] [--graph] [--out results/decode_loop.json]
"""

from __future__ import annotations

import argparse
import dataclasses
import json
import pathlib
import statistics
import sys
import time

sys.path.insert(0, str(pathlib.Path(__file__).resolve().parent.parent))

import torch  # noqa: E402

from pagedattn import (LLAMA3_8B, LLAMA3_70B, QWEN25_05B, allocate, flat_splits_for,  # noqa: E402
                       flat_waves_per_simd, plan_launch)
from pagedattn.cache_ops import reshape_and_cache  # noqa: E402
from pagedattn.hip_decode import _cu_count, paged_decode_hip  # noqa: E402

SHAPES = {"llama3-8b": LLAMA3_8B, "llama3-70b": LLAMA3_70B, "qwen2.5-0.5b": QWEN25_05B}
TOKENS_PER_PAGE = 16


@dataclasses.dataclass
class Result:
    """The reference's Result fields (bench_vllm.py:43-61), for the attention share."""

    backend: str
    model: str
    requests: int
    prompt_tokens: int
    output_tokens: int
    wall_s: float
    tpot_ms_p50: float
    tpot_ms_p90: float
    tpot_ms_p99: float
    ttft_ms_p50: float
    output_tok_per_s: float
    total_tok_per_s: float
    slo_attainment: dict[str, float]
    tpot_source: str
    max_model_len: int
    gpu_memory_utilization: float
    note: str = ""


def run(args, keep_state: bool = False):
    """Run the loop; returns the Result, or (Result, layers, launch) with
    `keep_state` (layers: (cache, slots, q, kv, out) per layer, caches at the
    lengths of the last step; launch: the decode's launch keywords)."""
    if not torch.cuda.is_available():
        raise SystemExit("bench_decode_loop needs a GPU: the HIP decode has no CPU path")
    dev = torch.device("cuda:0")
    shape = SHAPES[args.shape]
    b, p, n, w = args.requests, args.prompt, args.output_tokens, args.warmup
    total = p + w + n
    sdt = torch.float32 if args.kv == "int8" else torch.float16
    row_dtype = torch.bfloat16 if args.kv == "bf16" else torch.float16
    g = torch.Generator(device="cuda").manual_seed(args.seed)

    # one pool per layer, filled for every position the loop will reach
    lens = torch.full((b,), p, dtype=torch.int32, device=dev)  # each step adds one first
    layers = []
    for layer in range(args.layers):
        c = allocate(shape, b, [total] * b, block_size=TOKENS_PER_PAGE, kv_dtype=args.kv, device="cuda",
                     seed=args.seed + layer, scale_dtype=sdt, fill_device="cuda")
        c = dataclasses.replace(c, seq_lens=lens)  # every layer sees the same lengths
        # slot of position p + s of sequence r: page bt[r, pos // 16], row pos % 16
        pos = torch.arange(p, total, device=dev)
        pages = c.block_table.long()[:, pos // TOKENS_PER_PAGE]          # [b, w + n]
        slots = (pages * TOKENS_PER_PAGE + (pos % TOKENS_PER_PAGE)).t().contiguous()  # [w + n, b]
        q = torch.randn((b, shape.num_q_heads, shape.head_dim), generator=g, device=dev).to(row_dtype)
        kv = torch.randn((2, b, shape.num_kv_heads, shape.head_dim), generator=g, device=dev).to(row_dtype)
        layers.append((c, slots, q, kv, torch.empty_like(q)))

    wps = flat_waves_per_simd(args.kv, shape.head_dim, sdt if args.kv == "int8" else None)
    # one launch for the whole run, planned as the vLLM boundary plans a step
    # (batch size and the longest length the run reaches, no host lengths)
    flat = flat_splits_for(shape.num_kv_heads, shape.gqa_group, _cu_count(dev), wps, args.kv)
    mode = getattr(args, "launch", "plan")
    if mode == "flat":
        launch = {"flat_splits": flat}
    elif mode == "unsplit":
        launch = {"num_splits": 1, "max_seq_len": total}
    else:
        launch = plan_launch(b, total, shape.num_kv_heads, shape.gqa_group, _cu_count(dev), wps,
                             kv_dtype=args.kv, head_dim=shape.head_dim).launch_kwargs()
    counters = {"decode_calls": 0, "decode_tokens": 0, "delegated_calls": 0}

    def step(s: int) -> None:
        # the new token is at position p + s; it is written and then attended
        # to, so the decode sees p + s + 1 tokens (as vLLM's seq_lens does)
        lens.add_(1)
        for c, slots, q, kv, out in layers:
            reshape_and_cache(kv[0], kv[1], c, slots[s])
            paged_decode_hip(q, c, out=out, **launch)
            counters["decode_calls"] += 1
            counters["decode_tokens"] += b

    for s in range(w):
        step(s)
    torch.cuda.synchronize()
    counters.update(decode_calls=0, decode_tokens=0)
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    if args.graph:
        # One step as a HIP graph: the step index lives on the device, and
        # each layer's slot row is selected from it inside the graph, so a
        # replay needs no host work. Capture records without running.
        idx = torch.full((1,), w, dtype=torch.long, device=dev)
        cur = [torch.empty((1, b), dtype=torch.long, device=dev) for _ in layers]

        def graph_step() -> None:
            lens.add_(1)
            for (c, slots, q, kv, out), slot in zip(layers, cur):
                torch.index_select(slots, 0, idx, out=slot)
                reshape_and_cache(kv[0], kv[1], c, slot[0])
                paged_decode_hip(q, c, out=out, **launch)
            idx.add_(1)

        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            graph_step()
        torch.cuda.synchronize()

        def timed(i: int) -> None:
            graph.replay()
            counters["decode_calls"] += len(layers)
            counters["decode_tokens"] += b * len(layers)
    else:
        def timed(i: int) -> None:
            step(w + i)
    check_each = getattr(args, "check_each", False)
    t0 = time.perf_counter()
    for i, (e0, e1) in enumerate(events):
        e0.record()
        timed(i)
        e1.record()
        if check_each:
            # every step (every replay) against an eager decode of the same state
            torch.cuda.synchronize()
            for c, _, q, _, out in layers:
                if not torch.equal(out, paged_decode_hip(q, c, **launch)):
                    raise RuntimeError(f"step {i}: output differs from an eager decode of the same state")
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    tpot = sorted(e0.elapsed_time(e1) for e0, e1 in events)

    # the counters must show that this library's decode served every step
    if counters["decode_calls"] != n * args.layers or counters["delegated_calls"]:
        raise RuntimeError(f"decode counters {counters} do not cover the {n} x {args.layers} timed calls")
    print(f"  [decode] {counters['decode_calls']:,} calls over {counters['decode_tokens']:,} tokens, "
          f"launch {launch}, none delegated")

    # self-check on the last step (the lengths are still the ones it decoded):
    # the timed launch against the other one (flat or unsplit), and bit
    # stability
    c, _, q, _, out = layers[-1]
    a = paged_decode_hip(q, c, **launch).clone()
    a2 = paged_decode_hip(q, c, **launch)
    other = {"flat_splits": flat} if "flat_splits" not in launch else {"num_splits": 1}
    ref = paged_decode_hip(q, c, **other)
    torch.cuda.synchronize()
    # each launch rounds its fp32 result to the fp16/bf16 output on its own,
    # so besides the 2e-3 they may differ by an output ulp (<= 2^-10 |ref|
    # for fp16; 2^-7 for bf16)
    ulp = 2.0 ** -7 if ref.dtype == torch.bfloat16 else 2.0 ** -10
    diff = (a.float() - ref.float()).abs()
    err = diff.max().item()
    excess = (diff - ulp * ref.float().abs()).max().item()
    if not torch.equal(a, a2) or excess >= 2e-3 or not torch.equal(a, out):
        raise RuntimeError(f"self-check failed: max |{launch} - {other}| = {err:.2e}, bit-stable "
                           f"{torch.equal(a, a2)}, equal to the timed step {torch.equal(a, out)}")

    def pct(x: float) -> float:
        return tpot[min(len(tpot) - 1, int(round(x * (len(tpot) - 1))))]

    result = Result(
        backend="pagedattn-hip (attention only)",
        model=f"{args.shape} attention, {args.layers} layers, {args.kv} KV",
        requests=b,
        prompt_tokens=b * p,
        output_tokens=b * n,
        wall_s=wall,
        tpot_ms_p50=statistics.median(tpot),
        tpot_ms_p90=pct(0.90),
        tpot_ms_p99=pct(0.99),
        ttft_ms_p50=float("nan"),
        output_tok_per_s=b * n / wall,
        total_tok_per_s=b * n / wall,
        slo_attainment={f"{x:g}ms": sum(1 for t in tpot if t <= x) / len(tpot)
                        for x in [float(v) for v in args.slo.split(",") if v]},
        tpot_source=("HIP events around each step's KV writes and decodes (all layers)"
                     + (", one HIP graph replay per step" if args.graph else ", eager launches")),
        max_model_len=total,
        gpu_memory_utilization=float("nan"),
        note=f"no weights, MLP, sampling or prefill; launch {launch}; self-check against {other}: "
             f"max abs diff {err:.2e}",
    )
    return (result, layers, launch) if keep_state else result


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--shape", default="llama3-8b", choices=sorted(SHAPES))
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--requests", type=int, default=64)
    ap.add_argument("--prompt", type=int, default=4096)
    ap.add_argument("--output-tokens", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--kv", default="fp16", choices=["fp16", "bf16", "fp8_e5m2", "int8"])
    ap.add_argument("--slo", default="10,20,50,100")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--graph", action="store_true", help="replay each step as one HIP graph")
    ap.add_argument("--launch", default="plan", choices=["plan", "flat", "unsplit"],
                    help="plan: as the vLLM boundary plans the step (default); or force one launch")
    ap.add_argument("--out", default=None, help="append the run to this JSON file ({'runs': [...]})")
    args = ap.parse_args()
    if args.output_tokens < 1 or args.prompt < 1 or args.requests < 1 or args.layers < 1:
        raise SystemExit("--output-tokens, --prompt, --requests and --layers must be positive")
    if args.graph and args.warmup < 1:
        raise SystemExit("--graph needs --warmup >= 1 (the split workspace is allocated before capture)")

    r = run(args)
    print(f"backend            {r.backend}")
    print(f"model              {r.model}")
    print(f"requests           {r.requests}  (prompt {args.prompt}, {args.output_tokens} output tokens each)")
    print(f"TPOT p50/p90/p99   {r.tpot_ms_p50:.3f} / {r.tpot_ms_p90:.3f} / {r.tpot_ms_p99:.3f} ms")
    print(f"TPOT source        {r.tpot_source}")
    print(f"output throughput  {r.output_tok_per_s:,.0f} tok/s (attention only)")
    print("SLO attainment     " + "  ".join(f"{k}:{v*100:.0f}%" for k, v in r.slo_attainment.items()))
    print(json.dumps(dataclasses.asdict(r)))
    if args.out:
        out = pathlib.Path(args.out)
        out.parent.mkdir(parents=True, exist_ok=True)
        runs = []
        if out.exists():
            try:
                runs = json.loads(out.read_text(encoding="utf-8")).get("runs", [])
            except (ValueError, AttributeError):
                runs = []
        runs.append(dataclasses.asdict(r))
        out.write_text(json.dumps({"runs": runs}, indent=2), encoding="utf-8")
        print(f"wrote {out}  ({len(runs)} run(s) recorded)")


if __name__ == "__main__":
    main()
