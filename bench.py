"""Benchmark of the paged decode attention hot path on one MI355X.

Workload (default): Qwen2.5-7B-shape paged decode — 64 sequences, 28 query /
4 KV heads (GQA 7), head_dim 128, block 16, bf16, context U{512..4096}, block
tables drawn from a random permutation of a pool 1.25x the blocks needed,
q/K/V ~ N(0, 1) (synthetic: random values, no checkpoint). One step = one
decode-attention call for the whole batch (one layer). The schedule is the
seam's: for a batch with at least one (sequence, KV head) unit per CU, or
block tables holding 16 tiles per CU (C2, C3), the planned one --
ir_paged_decode_plan builds the balanced schedule of the
batch's metadata once per decode step and every layer runs
ir_paged_decode_planned on it, so the timed loop rebuilds a plan every
``--layers`` (28) calls -- otherwise ir_paged_decode's fixed split-KV
partitions (``--schedule`` forces either).

Timing: W warm-up calls, then K calls captured in one hipGraph and replayed
between two events on the launch stream, with torch.cuda.synchronize() on
both sides. Calls rotate over R disjoint copies of the pool + block tables so
consecutive calls do not hit K/V left in the 256 MB MALL by the previous one.
``roofline.peak`` is the published MI355X figure (8 TB/s HBM, 2.5 PFLOP/s dense
bf16 MFMA) and ``frac`` is taken against it; ``roofline.measured_peak`` is the
same roof measured on the device after the timing (a 1 GiB device copy, or an
8192^3 bf16 matmul through torch's BLAS), reported beside it.
``value`` is per call with the plan builds included; the roofline's
``achieved`` is the attention kernel's own launches (a graph of K runs
without plan builds).

Other workloads (``--workload``): ``prefill`` -- 8 sequences x 512-token
chunks after cached prefixes of up to 8192 tokens (pairs sharing prefix
blocks), one call of the chunked-prefill MFMA kernel per step, value in
TFLOP/s of unmasked (query, key) pairs; ``mixed`` -- one 28-layer engine step
of 224 decode rows (context U{256..4096}) + 4 x 256-token prefill chunks
(scatter + decode + prefill per layer) replayed as one hipGraph, value in us
per step; ``rope`` -- the fused rotary embedding + KV scatter of one such step's
layer (1,248 new tokens, 28 q / 4 kv heads), value in GB/s of algorithmic bytes.

Prints one JSON line: value = achieved KV GB/s (algorithmic bytes sum(ctx) *
2 * H_kv * D * 2 per call / time per call), plus us_per_call, a roofline
object for the decode kernel and the CPU baseline: the oracle's restatement of
the reference naive-gather fallback (gather -> repeat_kv -> masked softmax,
in bf16 like the reference) timed on the host cores on the same inputs.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import torch

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E, published
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, published
METRIC = "paged decode attn µs/call + achieved KV HBM GB/s (% of peak), Qwen2.5-7B shape"


def _parse() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--workload", choices=("decode", "prefill", "mixed", "rope"), default="decode")
    p.add_argument("--config", default=None, help="decode: qwen7b-bf16 (default) | qwen0.5b-fp32 | qwen7b-skewed")
    p.add_argument("--rotations", type=int, default=3)
    p.add_argument("--partition", type=int, default=0, help="split-KV partition tokens (0 = library default)")
    p.add_argument("--schedule", choices=("auto", "planned", "fixed"), default="auto",
                   help="decode: the seam's choice (default: kernels.decode_plan_pays), "
                   "balanced plan + run, or fixed split-KV partitions; prefill: the seam's choice "
                   "(kernels.prefill_plan_pays), the work plan, or none")
    p.add_argument("--layers", type=int, default=28,
                   help="calls per decode / prefill plan (layers of one step sharing its metadata)")
    p.add_argument("--cpu-iters", type=int, default=5, help="timed CPU-baseline iterations (0 = skip)")
    p.add_argument("--cpu-seqs", type=int, default=0, help="sequences in the CPU sample (0 = all)")
    p.add_argument("--check", action="store_true", help="also check the output against the oracle")
    p.add_argument("--mode", choices=("graph", "eager"), default="graph",
                   help="time a hipGraph replay of the K calls (default) or host-launched calls")
    p.add_argument("--overlap", action="store_true",
                   help="mixed: decode and prefill on two streams (default: one stream, measured faster)")
    p.add_argument("--copy-calib-mib", type=int, default=0,
                   help="after timing, run 10 device copies of this many MiB (counter calibration)")
    return p.parse_args()


WARM_MS = 50.0  # GPU time of graph replays before the timed ones
TIMED_REPLAYS = 7  # timed replays; the median is reported
_REPLAY_STATS: dict[str, dict] = {}


def _graph_ms(fn, steps: int, tag: str = "call") -> float:
    """ms per call of ``steps`` calls of fn captured in one hipGraph.

    The graph is replayed until at least ``WARM_MS`` of GPU time has passed
    (clocks and caches reach their steady state), then ``TIMED_REPLAYS``
    replays are timed one by one between events on the launch stream; the
    median per-call time is returned and the spread kept under ``tag``."""
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        fn(0)
    torch.cuda.current_stream().wait_stream(stream)
    with torch.cuda.graph(graph):
        for i in range(steps):
            fn(i)
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    warm_ms, warm_replays = 0.0, 0
    while warm_ms < WARM_MS and warm_replays < 100000:
        s.record()
        graph.replay()
        e.record()
        torch.cuda.synchronize()
        warm_ms += s.elapsed_time(e)
        warm_replays += 1
    per_call = []
    for _ in range(TIMED_REPLAYS):
        s.record()
        graph.replay()
        e.record()
        torch.cuda.synchronize()
        per_call.append(s.elapsed_time(e) / steps)
    _REPLAY_STATS[tag] = {
        "timed_replays": TIMED_REPLAYS,
        "calls_per_replay": steps,
        "warm_replays": warm_replays,
        "warm_ms": round(warm_ms, 2),
        "min_us": round(min(per_call) * 1e3, 3),
        "max_us": round(max(per_call) * 1e3, 3),
    }
    return statistics.median(per_call)


def _eager_ms(fn, steps: int) -> float:
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for i in range(steps):
        fn(i)
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / steps


def _gpu_decode(case, args):
    """Times the decode calls. Returns (info, eager_ms, call_ms, kernel_ms, outs):
    call_ms per decode call (planned: one plan build every ``--layers`` calls,
    as one decode step's layers share it), kernel_ms per launch of the dominant
    (attention) kernel alone."""
    from infrared_amd import kernels

    cfg = case.config
    dev = case.q.device
    b, max_blocks = cfg.num_seqs, case.block_tables[0].shape[1]
    hq, hkv, bs = cfg.num_q_heads, cfg.num_kv_heads, cfg.block_size
    rot = len(case.block_tables)
    outs = [torch.empty_like(case.q) for _ in case.block_tables]
    if args.schedule == "auto":
        planned = kernels.decode_plan_pays(b, hq, hkv, max_blocks, bs, dev)
    else:
        planned = args.schedule == "planned" and kernels.decode_plan_bytes(b, hq, hkv, max_blocks, bs) > 0
    info = {"schedule": "planned" if planned else "fixed"}
    if planned:
        plans = [kernels.decode_plan(bt, case.context_lens, hq, case.k_cache, bs) for bt in case.block_tables]
        ws_bytes = kernels.planned_workspace_bytes(b, hq, hkv, cfg.head_dim)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        ctr = torch.zeros(kernels.decode_num_counters(b, hq, hkv), dtype=torch.int32, device=dev)

        def run(i: int) -> None:
            r = i % rot
            kernels.paged_decode_planned(case.q, case.k_cache, case.v_cache, plans[r], cfg.scale, out=outs[r],
                                         workspace=ws, counters=ctr)

        def plan(i: int) -> None:
            p = i % rot
            kernels.decode_plan(case.block_tables[p], case.context_lens, hq, case.k_cache, bs, buf=plans[p].buf)

        def call(i: int) -> None:
            if i % args.layers == 0:
                plan(i // args.layers)
            run(i)

        info.update({"layers_per_plan": args.layers, "plan_bytes": int(plans[0].buf.numel()),
                     "workspace_bytes": ws_bytes})
    else:
        part = args.partition or kernels.default_partition(b, hkv, max_blocks, bs)
        ws_bytes = kernels.decode_workspace_bytes(b, hq, hkv, cfg.head_dim, max_blocks, bs, part)
        ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=dev)
        ctr = torch.zeros(kernels.decode_num_counters(b, hq, hkv), dtype=torch.int32, device=dev)

        def call(i: int) -> None:
            r = i % rot
            kernels.paged_decode(case.q, case.k_cache, case.v_cache, case.block_tables[r], case.context_lens,
                                 bs, cfg.scale, out=outs[r], partition_tokens=part, workspace=ws, counters=ctr)

        run = call
        info.update({"partition_tokens": part, "workspace_bytes": ws_bytes})

    for i in range(args.warmup):
        call(i)
    torch.cuda.synchronize()
    eager_ms = _eager_ms(call, args.steps)
    if args.mode == "eager":
        return info, eager_ms, eager_ms, eager_ms, outs
    call_ms = _graph_ms(call, args.steps, "call")
    kernel_ms = _graph_ms(run, args.steps, "kernel") if planned else call_ms
    if planned:
        info["plan_us"] = round(_graph_ms(plan, max(args.steps // 4, 8), "plan") * 1e3, 2)
    return info, eager_ms, call_ms, kernel_ms, outs


def _cpu_host() -> dict:
    """Host facts for the CPU baseline: the threads torch uses (the box's CPU
    share: OMP_NUM_THREADS), the CPUs the OS reports and the CPU model."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = None
    return {"cores": torch.get_num_threads(), "host_cpus": os.cpu_count(), "affinity_cpus": affinity,
            "cpu_model": model}


def _cpu_median(fn, iters: int) -> tuple[float, float, float]:
    """(median, min, max) seconds of ``iters`` timed calls of fn after one warm-up."""
    fn()
    times = []
    for _ in range(iters):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), min(times), max(times)


def _cpu_baseline(case, args):
    """The reference's naive-gather fallback (the oracle's restatement of
    gather -> repeat_kv -> masked softmax, in the workload dtype) on the host
    cores over the same inputs. ``executed_bytes``: the padded, repeated K/V the
    naive path's two einsums read (B * T_max * H_q * D * 2 tensors)."""
    from oracle import naive as O

    cfg = case.config
    n = args.cpu_seqs or cfg.num_seqs
    bt = case.block_tables[0][:n].cpu()
    ctx = case.context_lens[:n].cpu().tolist()
    tables = [row.tolist() for row in bt]
    t_max = max(ctx)
    gs = O.decode_gather_slots(tables, ctx, cfg.block_size, t_max)
    mask = O.decode_mask(ctx, t_max, cfg.dtype)
    q = case.q[:n, None].cpu()
    kc, vc = case.k_cache.cpu(), case.v_cache.cpu()
    host = _cpu_host()
    t, t_lo, t_hi = _cpu_median(lambda: O.paged_attention_naive(q, kc, vc, gs, mask, cfg.scale, cfg.n_rep),
                                args.cpu_iters)
    esize = torch.tensor([], dtype=cfg.dtype).element_size()
    kv = sum(ctx) * 2 * cfg.num_kv_heads * cfg.head_dim * esize
    executed = n * t_max * cfg.num_q_heads * cfg.head_dim * esize * 2
    return {
        "value": round(kv / t / 1e9, 4),
        "unit": "GB/s",
        "us_per_call": round(t * 1e6, 1),
        "min_us": round(t_lo * 1e6, 1),
        "max_us": round(t_hi * 1e6, 1),
        **host,
        "kind": "port",
        "algorithmic_bytes": kv,
        "executed_bytes": executed,
        "executed_over_algorithmic": round(executed / kv, 2),
        "sample": f"{n} of {cfg.num_seqs} sequences (sum ctx {sum(ctx)}, padded to {t_max}), naive gather+"
        f"repeat_kv+masked softmax in {str(cfg.dtype).replace('torch.', '')}, median of {args.cpu_iters} "
        "after 1 warm-up, torch CPU",
    }


def _traffic(name: str) -> tuple[int | None, str | None]:
    """HBM bytes per launch of a kernel/workload measured with rocprofv3 counters, if recorded."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"{name}_traffic.json")
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        rec = json.load(f)
    return int(rec["hbm_bytes_per_launch"]), os.path.relpath(path, os.path.dirname(path) + "/..")


def _bench_prefill(args) -> dict:
    """8 x 512-token chunks after cached prefixes: one prefill call per step."""
    from infrared_amd import kernels
    from infrared_amd.workloads import make_prefill_case

    case = make_prefill_case("qwen7b-prefill", "cuda", rotations=args.rotations)
    cfg = case.config
    out = torch.empty_like(case.q)
    total_q, max_blocks = case.q.shape[0], case.block_tables[0].shape[1]
    # the work plan (the seam's choice unless --schedule forces it), rebuilt
    # every --layers calls as an engine step would
    planned = args.schedule == "planned" or (args.schedule == "auto" and kernels.prefill_plan_pays(
        cfg.num_seqs, cfg.chunk, cfg.num_q_heads, cfg.num_kv_heads))
    plan_buf = torch.empty(max(256, kernels.prefill_plan_bytes(cfg.num_seqs, cfg.chunk, cfg.num_q_heads,
                                                               cfg.num_kv_heads, cfg.head_dim)),
                           dtype=torch.uint8, device="cuda")
    plan = [None]

    def call(i: int) -> None:
        if planned and i % args.layers == 0:
            plan[0] = kernels.prefill_plan(case.cu_seqlens_q, case.q_start, total_q, cfg.chunk, max_blocks,
                                           cfg.block_size, cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim,
                                           buf=plan_buf)
        kernels.paged_prefill(case.q, case.k_cache, case.v_cache, case.block_tables[i % len(case.block_tables)],
                              case.cu_seqlens_q, case.q_start, cfg.chunk, cfg.block_size, cfg.scale, out=out,
                              plan=plan[0])

    ms = _time_graph(call, args) if args.mode == "graph" else _time_eager(call, args)
    if args.copy_calib_mib > 0:
        _copy_calibration(args.copy_calib_mib)
    tflops = case.flops / (ms * 1e-3) / 1e12
    cpu = None
    if args.cpu_iters > 0:
        from oracle import naive as O

        # bounded sample: the reference's naive path for one chunk (sequence 0)
        b = 0
        n, pre = case.q_lens[b], case.prefixes[b]
        row = case.block_tables[0][b].cpu().tolist()
        gs = torch.tensor([[O.slot(row, p, cfg.block_size) for p in range(pre + n)]])
        mask = O.attention_mask([0], pre, n, pre + n, cfg.dtype)
        q = case.q[None, :n].cpu()
        kc, vc = case.k_cache.cpu(), case.v_cache.cpu()
        t, t_lo, t_hi = _cpu_median(lambda: O.paged_attention_naive(q, kc, vc, gs, mask, cfg.scale, cfg.n_rep),
                                    args.cpu_iters)
        fl = 4 * cfg.num_q_heads * cfg.head_dim * (n * pre + n * (n + 1) // 2)
        # the naive path computes every (query, key) pair of the padded score matrix
        fl_exec = 4 * cfg.num_q_heads * cfg.head_dim * n * (pre + n)
        cpu = {"value": round(fl / t / 1e12, 6), "unit": "TFLOP/s", "us_per_call": round(t * 1e6, 1),
               "min_us": round(t_lo * 1e6, 1), "max_us": round(t_hi * 1e6, 1), **_cpu_host(), "kind": "port",
               "algorithmic_flops": fl, "executed_flops": fl_exec,
               "sample": f"sequence 0 only ({n} queries after a {pre}-token prefix), naive gather+repeat_kv+masked "
               f"softmax in bf16, median of {args.cpu_iters} after 1 warm-up, torch CPU"}
    return {
        "metric": "paged prefill TFLOP/s (unmasked pairs), 8 x 512-token chunks after cached prefixes, Qwen2.5-7B shape",
        "value": round(tflops, 2), "unit": "TFLOP/s", "us_per_call": round(ms * 1e3, 2),
        "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"{cfg.name}: {cfg.num_seqs} chunks of {cfg.chunk} after prefixes {case.prefixes}, "
                   f"{cfg.num_q_heads}q/{cfg.num_kv_heads}kv heads, head_dim {cfg.head_dim}, block {cfg.block_size}",
                   "flops_per_call": case.flops, "kv_bytes_per_call": case.kv_bytes, "rotations": args.rotations,
                   "schedule": "work plan (heaviest first, heavy items cut)" if planned else "unplanned",
                   "layers_per_plan": args.layers if planned else None},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "measured_peak": _measured_peak("mfma"),
                     "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": _traffic("prefill_qwen7b-prefill")[0],
                     "timed": f"prefill call, {args.mode} launches, events on the launch stream"},
        "cpu_baseline": cpu,
    }


def _bench_mixed(args) -> dict:
    """One 28-layer mixed step (scatter + decode + prefill per layer) per graph replay."""
    from infrared_amd.mixed_step import MixedStep, make_mixed_case

    cfg, pool, batch, inputs = make_mixed_case("qwen7b-mixed", "cuda")
    step = MixedStep(pool, batch, inputs, cfg.scale, overlap=args.overlap)
    step.capture()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    warm_ms, warm = 0.0, 0
    while warm_ms < WARM_MS and warm < 1000:
        s.record()
        step.replay()
        e.record()
        torch.cuda.synchronize()
        warm_ms += s.elapsed_time(e)
        warm += 1
    n = max(TIMED_REPLAYS, args.steps // 20)
    per = []
    for _ in range(n):
        s.record()
        step.replay()
        e.record()
        torch.cuda.synchronize()
        per.append(s.elapsed_time(e))
    ms = statistics.median(per)
    _REPLAY_STATS["step"] = {"timed_replays": n, "warm_replays": warm, "warm_ms": round(warm_ms, 2),
                             "min_us": round(min(per) * 1e3, 2), "max_us": round(max(per) * 1e3, 2)}
    esize = 2
    dec_bytes = int(batch.dec_ctx.long().sum()) * 2 * cfg.num_kv_heads * cfg.head_dim * esize * cfg.num_layers
    pairs = cfg.num_prefill * (cfg.chunk * cfg.prefix + cfg.chunk * (cfg.chunk + 1) // 2)
    pre_flops = 4 * cfg.num_q_heads * cfg.head_dim * pairs * cfg.num_layers
    n_new = batch.write_slots.numel()
    scatter_bytes = 2 * n_new * cfg.num_kv_heads * cfg.head_dim * esize * 2 * cfg.num_layers
    gbps = dec_bytes / (ms * 1e-3) / 1e9
    cpu = None
    if args.cpu_iters > 0:
        from oracle import naive as O

        # bounded sample: one layer's decode rows through the reference's naive path
        nd = min(cfg.num_decode, 32)
        ctx = batch.dec_ctx[:nd].cpu().tolist()
        tables = [r.tolist() for r in batch.dec_tables[:nd].cpu()]
        t_max = max(ctx)
        gs = O.decode_gather_slots(tables, ctx, cfg.block_size, t_max)
        mask = O.decode_mask(ctx, t_max, cfg.dtype)
        q = inputs.q_dec[0, :nd, None].cpu()
        kc, vc = pool.k[0].cpu(), pool.v[0].cpu()
        n_rep = cfg.num_q_heads // cfg.num_kv_heads
        t, t_lo, t_hi = _cpu_median(lambda: O.paged_attention_naive(q, kc, vc, gs, mask, cfg.scale, n_rep),
                                    args.cpu_iters)
        kvb = sum(ctx) * 2 * cfg.num_kv_heads * cfg.head_dim * esize
        executed = nd * t_max * cfg.num_q_heads * cfg.head_dim * esize * 2
        cpu = {"value": round(kvb / t / 1e9, 4), "unit": "GB/s", "us_per_call": round(t * 1e6, 1),
               "min_us": round(t_lo * 1e6, 1), "max_us": round(t_hi * 1e6, 1), **_cpu_host(), "kind": "port",
               "algorithmic_bytes": kvb, "executed_bytes": executed,
               "sample": f"{nd} of {cfg.num_decode} decode rows of one layer (prefill and scatter not included; "
               f"x{cfg.num_layers} layers is an extrapolation), naive gather+repeat_kv+masked softmax in bf16, "
               f"median of {args.cpu_iters} after 1 warm-up, torch CPU"}
    return {
        "metric": "mixed engine step us per 28-layer hipGraph replay (224 decode rows + 4 x 256-token prefill chunks)",
        "value": round(ms * 1e3, 2), "unit": "us/step", "us_per_layer": round(ms * 1e3 / cfg.num_layers, 2),
        "ms_per_step": round(ms, 5), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"{cfg.name}: {cfg.num_layers} layers, {cfg.num_decode} decode rows ctx U"
                   f"[{cfg.decode_ctx_lo},{cfg.decode_ctx_hi}], {cfg.num_prefill} x {cfg.chunk}-token chunks, "
                   f"{cfg.num_q_heads}q/{cfg.num_kv_heads}kv heads, head_dim {cfg.head_dim}, block {cfg.block_size}",
                   "decode_kv_bytes_per_step": dec_bytes, "prefill_flops_per_step": pre_flops,
                   "scatter_bytes_per_step": scatter_bytes, "overlap_streams": args.overlap,
                   "replays": n},
        "roofline": {"bound": "hbm", "achieved": round(gbps, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "measured_peak": _measured_peak("hbm"),
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                     "timed": "whole step (decode KV bytes / step time: scatter and prefill time included)"},
        "cpu_baseline": cpu,
    }


def _bench_rope(args) -> dict:
    """Fused RoPE + KV scatter for one mixed-step layer: 1,248 tokens, 28 q / 4 kv heads."""
    from infrared_amd import kernels
    from oracle import naive as O

    n, hq, hkv, d, dtype = 1248, 28, 4, 128, torch.bfloat16
    num_slots = 1 << 20  # a 1 Mi-slot pool layer (2 GiB for K+V): writes land far apart
    g = torch.Generator(device="cuda").manual_seed(6)
    q = torch.randn(n, hq, d, generator=g, device="cuda").to(dtype)
    k = torch.randn(n, hkv, d, generator=g, device="cuda").to(dtype)
    v = torch.randn(n, hkv, d, generator=g, device="cuda").to(dtype)
    kc = torch.zeros(hkv, num_slots, d, dtype=dtype, device="cuda").permute(1, 0, 2)
    vc = torch.zeros_like(kc.permute(1, 0, 2)).permute(1, 0, 2)
    pos = torch.randint(0, 4096, (n,), generator=torch.Generator().manual_seed(6))
    cos, sin = (t.to("cuda") for t in O.rotary_cos_sin(pos, d, 1_000_000.0))
    slots = torch.randperm(num_slots, device="cuda")[:n]
    q_out = torch.empty_like(q)

    def call(i: int) -> None:
        kernels.rope_kv_scatter(q, k, v, cos, sin, kc, vc, slots, q_out=q_out)

    ms = _time_graph(call, args) if args.mode == "graph" else _time_eager(call, args)
    if args.copy_calib_mib > 0:
        _copy_calibration(args.copy_calib_mib)
    nbytes = (2 * n * hq * d + 4 * n * hkv * d) * 2 + 2 * n * d * 4 + n * 8
    gbps = nbytes / (ms * 1e-3) / 1e9
    return {
        "metric": "fused RoPE + KV scatter GB/s (1,248 tokens, 28q/4kv heads, head_dim 128)",
        "value": round(gbps, 2), "unit": "GB/s", "us_per_call": round(ms * 1e3, 3), "ms_per_step": round(ms, 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "one mixed-step layer: rotate q (in/out) and k, write k/v into a head-major pool",
                   "bytes_per_call": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(gbps, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "measured_peak": _measured_peak("hbm"),
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                     "timed": f"rope+scatter call, {args.mode} launches, events on the launch stream"},
        "cpu_baseline": None,
    }


def _measured_peak(bound: str) -> dict:
    """The roof the kernel is held against, measured on this device beside the
    published figure. HBM-bound kernels: a read-only stream of 4 GiB with the
    decode kernels' load form (``ir_hbm_read``: non-temporal 16-byte loads,
    ``value``) and a 1 GiB device-to-device copy (read + write bytes). MFMA-bound
    ones: an 8192^3 bf16 matmul through torch's BLAS. Events around 10 runs
    after 3 warm-ups; the buffers exceed the 256 MB MALL."""
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def rate(run, work):
        for _ in range(3):
            run()
        torch.cuda.synchronize()
        s.record()
        for _ in range(10):
            run()
        e.record()
        torch.cuda.synchronize()
        return round(work / (s.elapsed_time(e) / 10 * 1e-3), 1)

    if bound == "hbm":
        from infrared_amd import kernels

        src = torch.empty(4 << 30, dtype=torch.uint8, device="cuda")
        sink = torch.zeros(1, dtype=torch.int32, device="cuda")
        read = rate(lambda: kernels.hbm_read(src, sink), src.numel() / 1e9)
        del src
        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        copy = rate(lambda: dst.copy_(src), 2 * src.numel() / 1e9)
        del src, dst
        return {"value": read, "unit": "GB/s", "how": "4 GiB read-only stream (ir_hbm_read, non-temporal 16 B loads)",
                "copy": copy, "copy_how": "1 GiB device copy, read + write bytes"}
    n = 8192
    x = torch.randn(n, n, device="cuda", dtype=torch.bfloat16)
    y = torch.randn(n, n, device="cuda", dtype=torch.bfloat16)
    return {"value": rate(lambda: x @ y, 2 * n**3 / 1e12), "unit": "TFLOP/s", "how": "8192^3 bf16 matmul (torch BLAS)"}


def _time_eager(call, args) -> float:
    """ms per call over K host-launched calls after W warm-up calls."""
    for i in range(args.warmup):
        call(i)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for i in range(args.steps):
        call(i)
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / args.steps


def _copy_calibration(mib: int) -> None:
    """10 device copies of ``mib`` MiB: a known-size reference for the byte counters."""
    src = torch.empty(mib << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()


def _time_graph(call, args, tag: str = "call") -> float:
    """ms per call: W warm-up calls, then K calls captured in one hipGraph,
    warmed and timed as in :func:`_graph_ms`."""
    for i in range(args.warmup):
        call(i)
    torch.cuda.synchronize()
    return _graph_ms(call, args.steps, tag)


def main() -> int:
    args = _parse()
    if args.gpus != 1:
        print(
            f"bench.py measures the single-GPU hot path only; --gpus {args.gpus} is not supported "
            "(the decode kernel shards by sequence or KV head with no exchange inside attention)",
            file=sys.stderr,
        )
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    if args.workload != "decode":
        line = {"prefill": _bench_prefill, "mixed": _bench_mixed, "rope": _bench_rope}[args.workload](args)
        line.update({"n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "timing": dict(_REPLAY_STATS)})
        print(json.dumps(line), flush=True)
        return 0
    from infrared_amd.workloads import make_decode_case

    args.config = args.config or "qwen7b-bf16"
    case = make_decode_case(args.config, "cuda", rotations=args.rotations)
    cfg = case.config
    kv = case.kv_bytes
    info, eager_ms, graph_ms, kernel_ms, outs = _gpu_decode(case, args)
    us = graph_ms * 1e3
    gbps = kv / (graph_ms * 1e-3) / 1e9
    kgbps = kv / (kernel_ms * 1e-3) / 1e9
    check = None
    if args.check:
        from oracle import naive as O

        ref = O.decode_reference(
            case.q.cpu(), case.k_cache.cpu(), case.v_cache.cpu(), case.block_tables[0].cpu(),
            case.context_lens.cpu(), cfg.block_size, cfg.scale,
        )
        check = round((outs[0].float().cpu() - ref).abs().max().item(), 6)
    if args.copy_calib_mib > 0:
        _copy_calibration(args.copy_calib_mib)
    cpu = _cpu_baseline(case, args) if args.cpu_iters > 0 else None
    traffic, traffic_src = _traffic(f"decode_{'planned_' if info['schedule'] == 'planned' else ''}{args.config}")
    esize = torch.tensor([], dtype=cfg.dtype).element_size()
    line = {
        "metric": METRIC,
        "value": round(gbps, 2),
        "unit": "GB/s",
        "us_per_call": round(us, 2),
        "frac_of_hbm_peak": round(gbps / HBM_PEAK_GBPS, 4),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(graph_ms, 5),
        "eager_ms_per_step": round(eager_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": str(cfg.dtype).replace("torch.", "").replace("bfloat16", "bf16").replace("float32", "f32"),
        "data": "synthetic",
        "config": {
            "workload": f"{cfg.name} paged decode: {cfg.num_seqs} seqs, {cfg.num_q_heads}q/{cfg.num_kv_heads}kv "
            f"heads, head_dim {cfg.head_dim}, block {cfg.block_size}, ctx {cfg.ctx_kind}[{cfg.ctx_lo},{cfg.ctx_hi}]",
            "num_seqs": cfg.num_seqs,
            "sum_ctx": int(case.context_lens.long().sum()),
            "kv_bytes_per_call": kv,
            "rotations": args.rotations,
            **info,
            "bytes_per_token": 2 * cfg.num_kv_heads * cfg.head_dim * esize,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(kgbps, 2),
            "peak": HBM_PEAK_GBPS,
            "measured_peak": _measured_peak("hbm"),
            "unit": "GB/s",
            "frac": round(kgbps / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "kernel_us": round(kernel_ms * 1e3, 2),
            "timed": (f"{'paged_decode_planned_kernel' if info['schedule'] == 'planned' else 'paged_decode_kernel'}"
                      f" launches alone, {args.mode}, events on the launch stream"),
        },
        "cpu_baseline": cpu,
    }
    line["timing"] = dict(_REPLAY_STATS)
    if check is not None:
        line["max_abs_err_vs_fp32_oracle"] = check
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
