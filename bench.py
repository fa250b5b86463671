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
layer (1,248 new tokens, 28 q / 4 kv heads), value in GB/s of algorithmic bytes;
``engine`` -- the engine ladder rows (+HIP paged-attn, +hipGraph): a decode-heavy
burst through the seam with an attention-only model, value in output tok/s;
``reference-form`` -- the headline decode with the metadata unchanged reference
callers pass (gather_slots + mask), value in us per call; with ``--config
qwen7b-prefill`` the 8 x 512-token prefill in the reference's packed form
(gather_slots over every history + the varlen mask).

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
MFMA_F32_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix, published
METRIC = "paged decode attn µs/call + achieved KV HBM GB/s (% of peak), Qwen2.5-7B shape"


def _parse() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--workload", choices=("decode", "prefill", "mixed", "rope", "engine", "reference-form"),
                   default="decode")
    p.add_argument("--engine-batch", type=int, default=8, help="engine: sequences in the burst (max_batch)")
    p.add_argument("--config", default=None, help="decode: qwen7b-bf16 (default) | qwen0.5b-fp32 | qwen7b-skewed; reference-form: also qwen7b-prefill")
    p.add_argument("--rotations", type=int, default=3)
    p.add_argument("--partition", type=int, default=0, help="split-KV partition tokens (0 = library default)")
    p.add_argument("--schedule", choices=("auto", "planned", "fixed"), default="auto",
                   help="decode: the seam's choice (default: kernels.decode_plan_pays), "
                   "balanced plan + run, or fixed split-KV partitions; prefill: the seam's choice "
                   "(kernels.prefill_plan_pays), the work plan, or none")
    p.add_argument("--pairs", action="store_true",
                   help="decode: plan with share groups -- sequences 2i, 2i+1 whose block tables share prefix "
                   "blocks run as one unit per KV head, the shared blocks read once (--config qwen7b-pairs)")
    p.add_argument("--placement", choices=("global", "share-groups"), default="global",
                   help="prefill: the work plan's placement -- one global heaviest-first order, or each "
                   "(shared-prefix group, KV head) on one XCD (fewer bytes fetched)")
    p.add_argument("--dtype", choices=("bf16", "fp32"), default="bf16",
                   help="prefill: the chunks' dtype (fp32: the fp32 kernel, planned with IR_PLAN_F32)")
    p.add_argument("--layers", type=int, default=28,
                   help="calls per decode / prefill plan (layers of one step sharing its metadata)")
    p.add_argument("--cpu-iters", type=int, default=5, help="timed CPU-baseline iterations (0 = skip)")
    p.add_argument("--cpu-seqs", type=int, default=0, help="sequences in the CPU sample (0 = all)")
    p.add_argument("--check", action="store_true", help="also check the output against the oracle")
    p.add_argument("--mode", choices=("graph", "eager"), default="graph",
                   help="time a hipGraph replay of the K calls (default) or host-launched calls")
    p.add_argument("--layout", choices=("head_major", "slot_major"), default="head_major",
                   help="decode: the pool's physical layout -- head-major (default: a KV head's block is one "
                   "contiguous run) or the reference's contiguous [slots, H_kv, D] storage")
    p.add_argument("--separate-write", action="store_true",
                   help="mixed: the step's K/V write as its own launch (ir_kv_scatter) instead of inside the "
                        "prefill launch")
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
        plans = [kernels.decode_plan(bt, case.context_lens, hq, case.k_cache, bs, share_groups=args.pairs)
                 for bt in case.block_tables]
        ws_bytes = kernels.planned_workspace_bytes(b, hq, hkv, cfg.head_dim)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        ctr = torch.zeros(kernels.decode_num_counters(b, hq, hkv), dtype=torch.int32, device=dev)

        def run(i: int) -> None:
            r = i % rot
            kernels.paged_decode_planned(case.q, case.k_cache, case.v_cache, plans[r], cfg.scale, out=outs[r],
                                         workspace=ws, counters=ctr)

        def plan(i: int) -> None:
            p = i % rot
            kernels.decode_plan(case.block_tables[p], case.context_lens, hq, case.k_cache, bs, buf=plans[p].buf,
                                share_groups=args.pairs)

        def call(i: int) -> None:
            if i % args.layers == 0:
                plan(i // args.layers)
            run(i)

        info.update({"layers_per_plan": args.layers, "plan_bytes": int(plans[0].buf.numel()),
                     "workspace_bytes": ws_bytes, "pairs": bool(args.pairs),
                     "pairs_formed": int(plans[0].buf[:16].view(torch.int32)[3].item())})
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


def _gpu_scatter(case, args) -> dict:
    """The decode step's KV-slot scatter (``PagedKVPool.write``, reported beside
    the attention call): one new K and V row per sequence, at its last context
    position, through ``ir_kv_scatter``. The rows written are copies of what the
    pool already holds there, so the pool is left as it was."""
    from infrared_amd import kernels

    cfg = case.config
    bs = cfg.block_size
    pos = (case.context_lens.long() - 1).clamp(min=0)
    bt = case.block_tables[0].long()
    slots = bt.gather(1, (pos // bs)[:, None])[:, 0] * bs + pos % bs
    k_new, v_new = case.k_cache[slots].clone(), case.v_cache[slots].clone()

    def call(i: int) -> None:
        kernels.kv_scatter(case.k_cache, case.v_cache, k_new, v_new, slots)

    for i in range(args.warmup):
        call(i)
    torch.cuda.synchronize()
    ms = _graph_ms(call, args.steps, "scatter")
    esize = torch.tensor([], dtype=cfg.dtype).element_size()
    nbytes = 2 * cfg.num_seqs * cfg.num_kv_heads * cfg.head_dim * esize * 2
    return {"us_per_call": round(ms * 1e3, 3), "tokens": cfg.num_seqs, "bytes": nbytes,
            "GB_s": round(nbytes / (ms * 1e-3) / 1e9, 2),
            "timed": "ir_kv_scatter of the step's new K/V rows (one per sequence; read + write bytes), "
                     f"{args.mode} launches, events on the launch stream"}


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
    import dataclasses

    from infrared_amd import kernels
    from infrared_amd.workloads import PREFILL_CONFIGS, make_prefill_case

    f32 = args.dtype == "fp32"
    base = PREFILL_CONFIGS["qwen7b-prefill"]
    case = make_prefill_case(dataclasses.replace(base, dtype=torch.float32) if f32 else base, "cuda",
                             rotations=args.rotations)
    cfg = case.config
    out = torch.empty_like(case.q)
    total_q = case.q.shape[0]
    # the work plan (the seam's choice unless --schedule forces it), rebuilt
    # every --layers calls as an engine step would
    planned = args.schedule == "planned" or (args.schedule == "auto" and kernels.prefill_plan_pays(
        cfg.num_seqs, cfg.chunk, cfg.num_q_heads, cfg.num_kv_heads,
        max_keys=case.block_tables[0].shape[1] * cfg.block_size, dtype=cfg.dtype))
    plan_buf = torch.empty(max(256, kernels.prefill_plan_bytes(cfg.num_seqs, cfg.chunk, cfg.num_q_heads,
                                                               cfg.num_kv_heads, cfg.head_dim)),
                           dtype=torch.uint8, device="cuda")
    plan = [None]

    def call(i: int) -> None:
        if planned and i % args.layers == 0:
            bt = case.block_tables[i % len(case.block_tables)]
            plan[0] = kernels.prefill_plan(case.cu_seqlens_q, case.q_start, bt, total_q, cfg.chunk, cfg.block_size,
                                           cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim, buf=plan_buf,
                                           share_groups=args.placement == "share-groups", dtype=cfg.dtype)
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
               f"softmax in {args.dtype}, median of {args.cpu_iters} after 1 warm-up, torch CPU"}
    peak = MFMA_F32_PEAK_TFLOPS if f32 else MFMA_BF16_PEAK_TFLOPS
    traffic_name = ("prefill_f32_qwen7b-prefill" if f32 else "prefill_qwen7b-prefill") + (
        "" if args.placement == "global" else "-share-groups")
    return {
        "metric": "paged prefill TFLOP/s (unmasked pairs), 8 x 512-token chunks after cached prefixes, Qwen2.5-7B shape"
                  + (", fp32" if f32 else ""),
        "value": round(tflops, 2), "unit": "TFLOP/s", "us_per_call": round(ms * 1e3, 2),
        "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32" if f32 else "bf16", "data": "synthetic",
        "config": {"workload": f"{cfg.name}: {cfg.num_seqs} chunks of {cfg.chunk} after prefixes {case.prefixes}, "
                   f"{cfg.num_q_heads}q/{cfg.num_kv_heads}kv heads, head_dim {cfg.head_dim}, block {cfg.block_size}",
                   "flops_per_call": case.flops, "kv_bytes_per_call": case.kv_bytes, "rotations": args.rotations,
                   "schedule": "work plan (heaviest first, heavy items cut)" if planned else "unplanned",
                   "placement": args.placement if planned else None,
                   "layers_per_plan": args.layers if planned else None},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": peak, "unit": "TFLOP/s",
                     "measured_peak": _measured_peak("mfma", torch.float32 if f32 else torch.bfloat16),
                     "frac": round(tflops / peak, 4), "traffic": _traffic(traffic_name)[0],
                     "timed": f"prefill call, {args.mode} launches, events on the launch stream"},
        "cpu_baseline": cpu,
    }


def _bench_mixed(args) -> dict:
    """One 28-layer mixed step (K/V write, prefill and decode per layer) per graph replay."""
    from infrared_amd.mixed_step import MixedStep, make_mixed_case

    cfg, pool, batch, inputs = make_mixed_case("qwen7b-mixed", "cuda")
    step = MixedStep(pool, batch, inputs, cfg.scale, overlap=args.overlap, fused=not args.separate_write)
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
                   "kv_write": "own launch" if not step.fused else "inside the prefill launch",
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


class _AttnOnlyModel:
    """Embedding -> L x (attention + residual) -> output head, random weights, at
    a given attention shape: the engine flow's model for the ladder rows (the
    head is untied so greedy decoding does not just repeat the last token). The
    attention is the seam under measurement (``rope_paged_attention``: fused
    RoPE + KV write, then the paged kernels); projections are torch GEMMs.
    RoPE tables are built on the device from the step's positions (so a
    captured decode step rebuilds them on replay)."""

    def __init__(self, hid: int, hq: int, hkv: int, d: int, layers: int, vocab: int, theta: float, seed: int):
        g = torch.Generator().manual_seed(seed)
        self.shape = (hid, hq, hkv, d, layers, vocab, theta)
        self.emb = torch.randn(vocab, hid, generator=g) * 0.5
        self.w = [{"q": torch.randn(hid, hq * d, generator=g) / hid**0.5,
                   "k": torch.randn(hid, hkv * d, generator=g) / hid**0.5,
                   "v": torch.randn(hid, hkv * d, generator=g) / hid**0.5,
                   "o": torch.randn(hq * d, hid, generator=g) / (hq * d) ** 0.5} for _ in range(layers)]
        self.head = torch.randn(hid, vocab, generator=g) / hid**0.5
        self.gemb = self.emb.cuda().bfloat16()
        self.ghead = self.head.cuda().bfloat16()
        self.gw = [{n: t.cuda().bfloat16() for n, t in w.items()} for w in self.w]
        self.inv_freq = (1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))).cuda()

    def _rope(self, positions: torch.Tensor):
        freqs = positions.to(torch.float32)[..., None] * self.inv_freq
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos(), emb.sin()

    def forward(self, paged, tokens: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        """tokens / positions ``[B, S]`` on the device -> last-position logits ``[B, vocab]`` fp32."""
        from infrared_amd import rope_paged_attention

        hid, hq, hkv, d = self.shape[:4]
        b, s = tokens.shape
        x = self.gemb[tokens]
        cos, sin = self._rope(positions)
        for layer, w in enumerate(self.gw):
            q = (x @ w["q"]).view(b, s, hq, d)
            k = (x @ w["k"]).view(b, s, hkv, d)
            v = (x @ w["v"]).view(b, s, hkv, d)
            a = rope_paged_attention(q, k, v, cos, sin, paged, None, layer, d**-0.5, hq // hkv)
            x = x + a.reshape(b, s, hq * d) @ w["o"]
        return (x @ self.ghead).float()


def _engine_burst(model, prompts, new_tokens: int, pool, dec, tables):
    """One decode-heavy burst through the seam: a packed prefill step of every
    prompt, then greedy decode steps -- eager ``paged_attention`` calls, or
    replays of ``dec`` (a ``HipGraphDecoder`` on ``pool``) when given. Returns
    (tokens per sequence, last-position logits per step)."""
    from infrared_amd import metadata

    vocab = model.shape[5]
    b, plen = len(prompts), len(prompts[0])
    paged, _ = metadata.prefill_context(pool, tables, [0] * b, [plen] * b)
    toks = torch.tensor([t for p in prompts for t in p], device="cuda")[None]
    pos = torch.tensor([i for _ in prompts for i in range(plen)], device="cuda")[None]
    last = model.forward(paged, toks, pos)[0].view(b, plen, vocab)[:, -1]
    steps = [last]
    seqs = [list(p) for p in prompts]
    nxt = last.argmax(-1).tolist()
    for _ in range(new_tokens - 1):
        for sq, t in zip(seqs, nxt):
            sq.append(t)
        num_cached = [len(sq) - 1 for sq in seqs]
        if dec is not None:
            logits = dec.decode(tables, num_cached, [sq[-1] for sq in seqs])
        else:
            pg, _ = metadata.decode_context(pool, tables, num_cached)
            logits = model.forward(pg, torch.tensor([[sq[-1]] for sq in seqs], device="cuda"),
                                   torch.tensor(num_cached, device="cuda")[:, None])[:, -1]
        steps.append(logits.clone())  # (a replay's output is the graph's static buffer)
        nxt = logits.argmax(-1).tolist()
    for sq, t in zip(seqs, nxt):
        sq.append(t)
    return seqs, steps


def _engine_burst_cpu(model, prompts, new_tokens: int, tables):
    """The same burst on the host through the oracle's restatement of the
    reference's naive cached path (``PagedKVPool.write`` + gather + repeat_kv +
    masked softmax, ``infrared/model/triton_attention.py:110-129``), bf16:
    per-sequence prefill (``paged_engine.py:194-207``), batched decode with
    ``gather_slots`` + additive mask (``paged_engine.py:290-332``)."""
    from oracle import naive as O

    hid, hq, hkv, d, layers, vocab, theta = model.shape
    dt, bs = torch.bfloat16, 16
    nslots = (max(max(t) for t in tables) + 1) * bs
    kp = [torch.zeros(nslots, hkv, d, dtype=dt) for _ in range(layers)]
    vp = [torch.zeros(nslots, hkv, d, dtype=dt) for _ in range(layers)]
    w = [{n: t.to(dt) for n, t in wl.items()} for wl in model.w]
    emb, head = model.emb.to(dt), model.head.to(dt)

    def forward(tokens, positions, write, gs, mask):
        b, s = tokens.shape
        x = emb[tokens]
        cos, sin = O.rotary_cos_sin(positions, d, theta)
        for layer, wl in enumerate(w):
            q = (x @ wl["q"]).view(b, s, hq, d)
            k = (x @ wl["k"]).view(b, s, hkv, d)
            v = (x @ wl["v"]).view(b, s, hkv, d)
            q, k = O.apply_rotary_pos_emb(q, k, cos.to(dt), sin.to(dt))
            O.pool_write(kp[layer], vp[layer], k.reshape(-1, hkv, d), v.reshape(-1, hkv, d), write)
            a = O.paged_attention_naive(q, kp[layer], vp[layer], gs, mask, d**-0.5, hq // hkv)
            x = x + a.reshape(b, s, hq * d) @ wl["o"]
        return (x @ head).float()[:, -1]

    seqs = [list(p) for p in prompts]
    plen = len(prompts[0])
    nxt = []
    for sq, tb in zip(seqs, tables):
        slots = torch.tensor([O.slot(tb, p, bs) for p in range(plen)])
        logits = forward(torch.tensor([sq]), torch.arange(plen)[None], slots, slots[None],
                         O.attention_mask([0], 0, plen, plen, dt))
        nxt.append(int(logits[0].argmax()))
    for _ in range(new_tokens - 1):
        for sq, t in zip(seqs, nxt):
            sq.append(t)
        nc = [len(sq) - 1 for sq in seqs]
        ctx = [n + 1 for n in nc]
        write = torch.tensor([O.slot(tb, n, bs) for tb, n in zip(tables, nc)])
        gs = O.decode_gather_slots(tables, ctx, bs, max(ctx))
        logits = forward(torch.tensor([[sq[-1]] for sq in seqs]), torch.tensor(nc)[:, None], write, gs,
                         O.decode_mask(ctx, max(ctx), dt))
        nxt = logits.argmax(-1).tolist()
    for sq, t in zip(seqs, nxt):
        sq.append(t)
    return seqs


def _bench_engine(args) -> dict:
    """The engine ladder rows at the reference's throughput shape
    (``infrared/bench/harness.py:377-437`` ``measure``: a decode-heavy burst of
    ``max_batch`` 8-token prompts x 32 new tokens, output tok/s over the burst's
    wall time): "+HIP paged-attn" (eager seam every step) and "+hipGraph" (the
    decode step captured once per bucket and replayed), with an attention-only
    model at the Qwen2.5-7B attention shape (28 q / 4 kv heads, head_dim 128,
    hidden 3584) and random weights. Correctness: both rows generate the same
    tokens, and every step's logits match a CPU fp32 full recompute of the
    sequence within 2x the bf16-vs-fp32 error of the same recompute + 0.05."""
    b, plen, new = args.engine_batch, 8, 32
    layers = 4
    model = _AttnOnlyModel(3584, 28, 4, 128, layers, 1024, 1_000_000.0, seed=7)
    rng = torch.Generator().manual_seed(0)
    hid, hq, hkv, d, _, vocab, theta = model.shape
    prompts = torch.randint(1, 1024, (b, plen), generator=rng).tolist()
    per = -(-(plen + new) // 16)
    num_blocks = b * per + 8
    perm = torch.randperm(num_blocks, generator=rng).tolist()
    tables = [perm[i * per:(i + 1) * per] for i in range(b)]
    from infrared_amd import PagedKVPool
    from infrared_amd.hip_graph import HipGraphDecoder

    rows, outs = [], {}
    for tier, graph in (("+HIP paged-attn", False), ("+hipGraph", True)):
        pool = PagedKVPool(layers, num_blocks, 16, 4, 128, torch.bfloat16, device="cuda")
        dec = HipGraphDecoder(None, pool, max_num_seqs=b, t_max=plen + new, block_size=16,
                              step_fn=lambda buf, pg: model.forward(pg, buf.ids, buf.positions)[:, -1]) if graph else None
        _engine_burst(model, prompts, new, pool, dec, tables)  # warm-up (the graph row captures here)
        torch.cuda.synchronize()
        walls = []
        for _ in range(3):
            t0 = time.perf_counter()
            seqs, steps = _engine_burst(model, prompts, new, pool, dec, tables)
            torch.cuda.synchronize()
            walls.append(time.perf_counter() - t0)
        wall = statistics.median(walls)
        outs[tier] = (seqs, steps)
        rows.append({"tier": tier, "throughput_toks_per_s": round(b * new / wall, 1), "wall_s": round(wall, 4),
                     "timed_bursts": len(walls)})
    same = outs["+HIP paged-attn"][0] == outs["+hipGraph"][0]
    # CPU leg: the oracle's full recompute (fp32 and bf16) of each generated
    # sequence, teacher-forced, as the correctness reference and the baseline
    from oracle import naive as O

    def recompute(tokens, dtype):
        n = len(tokens)
        x = model.emb.to(dtype)[torch.tensor(tokens)][None]
        cos, sin = O.rotary_cos_sin(torch.arange(n)[None], d, theta)
        mask = O.attention_mask([0], 0, n, n, dtype)
        for w32 in model.w:
            w = {k_: t.to(dtype) for k_, t in w32.items()}
            q = (x @ w["q"]).view(1, n, hq, d)
            k = (x @ w["k"]).view(1, n, hkv, d)
            v = (x @ w["v"]).view(1, n, hkv, d)
            q, k = O.apply_rotary_pos_emb(q, k, cos, sin)
            a = O.masked_attention(q, O.repeat_kv(k, hq // hkv), O.repeat_kv(v, hq // hkv), mask, d**-0.5)
            x = x + a.reshape(1, n, hq * d) @ w["o"]
        return (x @ model.head.to(dtype))[0].float()

    seqs, steps = outs["+hipGraph"]
    worst = 0.0
    for i, sq in enumerate(seqs):
        want = recompute(sq, torch.float32)
        bf = recompute(sq, torch.bfloat16)
        got = torch.stack([st[i].cpu() for st in steps])  # logits at positions plen-1 .. plen+new-2
        rows_ = slice(plen - 1, plen - 1 + new)
        bar = 2 * (bf[rows_] - want[rows_]).abs().max().item() + 0.05
        worst = max(worst, (got - want[rows_]).abs().max().item() / bar)
    passed = same and worst <= 1.0
    for r in rows:
        r["correctness"] = {"passed": passed, "tokens_equal_across_rows": same,
                            "max_logit_err_over_bar": round(worst, 4)}
    cpu = None
    if args.cpu_iters > 0:
        t, t_lo, t_hi = _cpu_median(lambda: _engine_burst_cpu(model, prompts, new, tables), min(args.cpu_iters, 3))
        cpu_seqs = _engine_burst_cpu(model, prompts, new, tables)
        cpu = {"value": round(b * new / t, 2), "unit": "tok/s", "min_s": round(t_lo, 3), "max_s": round(t_hi, 3),
               **_cpu_host(), "kind": "port",
               "tokens_equal_to_gpu_rows": cpu_seqs == seqs,
               "sample": f"the same burst ({b} x {plen} + {new}) through the oracle's restatement of the "
               "reference's naive cached path in bf16 on the host, median of "
               f"{min(args.cpu_iters, 3)} after 1 warm-up"}
    graph_tps = rows[1]["throughput_toks_per_s"]
    return {
        "metric": "engine decode-heavy burst output tok/s (ladder rows +HIP paged-attn / +hipGraph)",
        "value": graph_tps, "unit": "tok/s", "ms_per_step": round(rows[1]["wall_s"] / new * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"{b} prompts x {plen} tokens, {new} greedy new tokens each; attention-only model, "
                   f"{layers} layers, 28q/4kv heads, head_dim 128, hidden 3584, vocab 1024, random weights, "
                   "block 16", "rows": rows},
        "roofline": None,
        "cpu_baseline": cpu,
    }


def _rows_ms(rows: dict, steps: int, per: int, warm: bool = True, prep=None) -> dict:
    """Median ms per call (a step's time / ``per``) of each row, the rows' steps
    interleaved (A, B, C, A, B, C, ...), after untimed rounds of at least
    ``WARM_MS`` of GPU time when ``warm``: the device's clock takes tens of
    milliseconds of sustained work to settle, so rows timed one after another
    would favour the later ones. ``prep`` runs before each step, outside the
    timed region."""
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    times = {name: [] for name in rows}
    warm_ms, timed = (0.0 if warm else WARM_MS), 0
    while timed < steps:
        for name, fn in rows.items():
            if prep is not None:
                prep()
            torch.cuda.synchronize()
            s.record()
            fn()
            e.record()
            torch.cuda.synchronize()
            if warm_ms < WARM_MS:
                warm_ms += s.elapsed_time(e)
            else:
                times[name].append(s.elapsed_time(e) / per)
        timed = min(len(v) for v in times.values())
    return {name: statistics.median(v) for name, v in times.items()}


def _bench_reference_form_prefill(args) -> dict:
    """Unchanged reference callers at the 8 x 512-token chunked-prefill shape:
    the step's metadata as the reference engine packs it for prefill and mixed
    steps (one frame: ``gather_slots [1, K]`` over every sequence's history +
    the varlen mask ``[1, 1, Q, K]``, ``infrared/engine/paged_engine.py:461-516``,
    no block tables) through ``paged_attention`` for ``--layers`` layers (KV
    write + attention per layer, eager launches). Rows: the seam recognising
    the packed form (one check per step) and running the chunked-prefill
    kernel; the same step with block-table fields filled by the caller; the
    mask kernel reading gather_slots + mask as given (``use_triton=False``,
    one step); and the form check alone."""
    from dataclasses import dataclass

    from infrared_amd import PagedContext, PagedKVPool, metadata, paged_attention
    from infrared_amd.workloads import make_prefill_case

    @dataclass(slots=True)
    class RefContext:  # the reference's PagedContext fields only
        pool: object
        write_slots: torch.Tensor
        gather_slots: torch.Tensor
        use_triton: bool = True

    case = make_prefill_case(args.config, "cuda")
    cfg = case.config
    hq, hkv, d, bs = cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim, cfg.block_size
    pool = PagedKVPool(1, case.pool_blocks, bs, hkv, d, cfg.dtype, device="cuda")
    pool.k[0].copy_(case.k_cache)
    pool.v[0].copy_(case.v_cache)
    nblk = [-(-(p + n) // bs) for p, n in zip(case.prefixes, case.q_lens)]
    tables = [row[:n].tolist() for row, n in zip(case.block_tables[0].cpu(), nblk)]
    ours, mask = metadata.prefill_context(pool, tables, case.prefixes, case.q_lens, with_mask=True)
    total = sum(case.q_lens)
    g = torch.Generator(device="cuda").manual_seed(2)
    q = case.q.view(1, total, hq, d)
    k = torch.randn(1, total, hkv, d, generator=g, device="cuda").to(cfg.dtype)
    v = torch.randn(1, total, hkv, d, generator=g, device="cuda").to(cfg.dtype)
    layers = args.layers
    fresh = []

    def step_ref():
        # a step's metadata arrives as new tensors, as the reference engine builds them
        gs, m = fresh.pop()
        paged = RefContext(pool, ours.write_slots, gs)
        for _ in range(layers):
            paged_attention(q, k, v, paged, m, 0, cfg.scale, cfg.n_rep)

    def step_ours():
        paged = PagedContext(pool, ours.write_slots, None, True, ours.block_tables, None, ours.cu_seqlens_q,
                             ours.q_start, ours.max_q_len)
        for _ in range(layers):
            paged_attention(q, k, v, paged, None, 0, cfg.scale, cfg.n_rep)

    def step_masked():
        paged = RefContext(pool, ours.write_slots, ours.gather_slots, use_triton=False)
        for _ in range(layers):
            paged_attention(q, k, v, paged, mask, 0, cfg.scale, cfg.n_rep)

    def check_only():
        gs, m = fresh.pop()
        pool.reference_varlen_form(gs, m)

    def prep():
        fresh.clear()
        fresh.append((ours.gather_slots.clone(), mask.clone()))

    ms = _rows_ms({"ref": step_ref, "ours": step_ours}, 15, layers, prep=prep)
    ms_ref, ms_ours = ms["ref"], ms["ours"]
    ms_check_ev = _rows_ms({"check": check_only}, 15, 1, prep=prep)["check"]
    # the check blocks the host until its record arrives, so the step waits
    # for its host wall time; events around a host-blocking call add their own
    # host overhead (reported beside it)
    host_ms = []
    for _ in range(15):
        prep()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        check_only()
        host_ms.append((time.perf_counter() - t0) * 1e3)
    ms_check = statistics.median(host_ms)
    form = pool._ref_varlen[1]
    ms_masked = _rows_ms({"masked": step_masked}, 1, layers, warm=False)["masked"]
    out_ref = paged_attention(q, k, v, RefContext(pool, ours.write_slots, ours.gather_slots), mask, 0, cfg.scale,
                              cfg.n_rep)
    out_ours = paged_attention(q, k, v, PagedContext(pool, ours.write_slots, None, True, ours.block_tables, None,
                                                     ours.cu_seqlens_q, ours.q_start, ours.max_q_len),
                               None, 0, cfg.scale, cfg.n_rep)
    torch.cuda.synchronize()
    tflops = case.flops / (ms_ref * 1e-3) / 1e12
    return {
        "metric": "chunked prefill attn us/call for unchanged reference callers (gather_slots + varlen mask), "
                  "8 x 512-token chunks",
        "value": round(ms_ref * 1e3, 2), "unit": "us/call", "ms_per_step": round(ms_ref * layers, 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"{cfg.name} in the reference's packed form: {len(case.q_lens)} chunks of "
                   f"{cfg.chunk} tokens after prefixes {case.prefixes}, {hq}q/{hkv}kv heads, head_dim {d}, block "
                   f"{bs}, gather_slots {tuple(ours.gather_slots.shape)}, mask {tuple(mask.shape)} "
                   f"({mask.numel() * mask.element_size() / 1e6:.0f} MB), {layers} layers per step (KV write + "
                   "attention per layer), eager",
                   "varlen_form_recognised": form is not None,
                   "equal_to_block_table_path": bool(torch.equal(out_ref, out_ours)),
                   "rows_us_per_call": {"reference form, recognised (one check per step)": round(ms_ref * 1e3, 2),
                                        "block-table fields from the caller": round(ms_ours * 1e3, 2),
                                        "mask kernel on gather_slots + mask": round(ms_masked * 1e3, 2)},
                   "form_check_us_per_step": round(ms_check * 1e3, 2),
                   "form_check_how": "host wall time of the call (it returns once the device's record is read), "
                                     "median of 15 after the event-timed rounds",
                   "form_check_event_us": round(ms_check_ev * 1e3, 2)},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None,
                     "timed": "whole call (KV write + attention, eager launches, the step's check amortised)"},
        "cpu_baseline": None,
    }


def _bench_reference_form(args) -> dict:
    """Unchanged reference callers at the Qwen2.5-7B decode shape: each step's
    metadata in the reference engine's own form (``gather_slots [B, T]`` +
    additive mask, ``infrared/engine/paged_engine.py:290-332``, no block
    tables; new tensors every step, made before the timed region) through
    ``paged_attention`` for ``--layers`` layers (KV write + attention per
    layer, eager launches). Rows: the seam recognising the decode form (one
    check per step, no host wait) and running the block-table kernels; the
    same layers captured as the reference's ``CudaGraphDecoder`` does; the
    same step with block-table fields filled by the caller; and the mask kernel
    reading gather_slots + mask as given (``use_triton=False``). The rows'
    steps are interleaved."""
    from dataclasses import dataclass

    from infrared_amd import PagedContext, PagedKVPool, kernels, metadata, paged_attention
    from infrared_amd.workloads import PREFILL_CONFIGS, make_decode_case

    if args.config in PREFILL_CONFIGS:
        return _bench_reference_form_prefill(args)

    @dataclass(slots=True)
    class RefContext:  # the reference's PagedContext fields only
        pool: object
        write_slots: torch.Tensor
        gather_slots: torch.Tensor
        use_triton: bool = True

    case = make_decode_case("qwen7b-bf16", "cuda")
    cfg = case.config
    b, hq, hkv, d, bs = cfg.num_seqs, cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim, cfg.block_size
    pool = PagedKVPool(1, case.pool_blocks, bs, hkv, d, cfg.dtype, device="cuda")
    pool.k[0].copy_(case.k_cache)
    pool.v[0].copy_(case.v_cache)
    ctx = case.context_lens.cpu().tolist()
    tables = [row[: -(-c // bs)].tolist() for row, c in zip(case.block_tables[0].cpu(), ctx)]
    ours, mask = metadata.decode_context(pool, tables, [c - 1 for c in ctx])
    g = torch.Generator(device="cuda").manual_seed(2)
    q = torch.randn(b, 1, hq, d, generator=g, device="cuda").to(cfg.dtype)
    k = torch.randn(b, 1, hkv, d, generator=g, device="cuda").to(cfg.dtype)
    v = torch.randn(b, 1, hkv, d, generator=g, device="cuda").to(cfg.dtype)
    layers, steps = args.layers, 15
    fresh = []

    def prep():
        # a step's metadata arrives as new tensors, as the reference engine
        # builds them (made before the timed region: the caller's work)
        fresh.clear()
        fresh.append((ours.gather_slots.clone(), mask.clone()))

    def step_ref():
        gs, m = fresh.pop()
        paged = RefContext(pool, ours.write_slots, gs)
        for _ in range(layers):
            paged_attention(q, k, v, paged, m, 0, cfg.scale, cfg.n_rep)

    def step_ours():
        paged = PagedContext(pool, ours.write_slots, ours.gather_slots, True, ours.block_tables, ours.context_lens)
        for _ in range(layers):
            paged_attention(q, k, v, paged, mask, 0, cfg.scale, cfg.n_rep)

    def step_masked():
        paged = RefContext(pool, ours.write_slots, ours.gather_slots, use_triton=False)
        for _ in range(layers):
            paged_attention(q, k, v, paged, mask, 0, cfg.scale, cfg.n_rep)

    # the reference's CudaGraphDecoder (infrared/engine/cuda_graph.py:263-285):
    # static gather_slots / mask, three warm-ups on a side stream, then the
    # step's layers captured; a replay re-checks the metadata on the device
    gs_s, m_s = ours.gather_slots.clone(), mask.clone()

    def forward_static():
        paged = RefContext(pool, ours.write_slots, gs_s)
        out = None
        for _ in range(layers):
            out = paged_attention(q, k, v, paged, m_s, 0, cfg.scale, cfg.n_rep)
        return out

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            forward_static()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_graph = forward_static()

    def step_graph():
        graph.replay()

    ms = _rows_ms({"ref": step_ref, "ours": step_ours, "graph": step_graph, "masked": step_masked}, steps, layers,
                  prep=prep)
    ms_ref, ms_ours, ms_masked, ms_graph = ms["ref"], ms["ours"], ms["masked"], ms["graph"]
    form = pool._ref_form[1]
    recognised = form is not None and form.verdict() is True  # (before another check takes the record)
    out_ref = paged_attention(q, k, v, RefContext(pool, ours.write_slots, ours.gather_slots), mask, 0, cfg.scale,
                              cfg.n_rep)
    out_ours = paged_attention(q, k, v, PagedContext(pool, ours.write_slots, ours.gather_slots, True,
                                                     ours.block_tables, ours.context_lens), mask, 0, cfg.scale,
                               cfg.n_rep)
    torch.cuda.synchronize()
    kv = case.kv_bytes
    return {
        "metric": "paged decode attn us/call for unchanged reference callers (gather_slots + mask), Qwen2.5-7B shape",
        "value": round(ms_ref * 1e3, 2), "unit": "us/call", "ms_per_step": round(ms_ref * layers, 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"{cfg.name} decode in the reference's metadata form: {b} seqs, {hq}q/{hkv}kv heads, "
                   f"head_dim {d}, block {bs}, gather_slots {tuple(ours.gather_slots.shape)}, {layers} layers per step "
                   "(KV write + attention per layer), eager",
                   "decode_form_recognised": recognised,
                   "equal_to_block_table_path": bool(torch.equal(out_ref, out_ours)),
                   "graph_replay_equal_to_block_table_path": bool(torch.equal(out_graph, out_ours)),
                   "rows_us_per_call": {"reference form, recognised (one check per step)": round(ms_ref * 1e3, 2),
                                        "reference form captured as the reference's CudaGraphDecoder does "
                                        "(check recorded, gating the mask kernel on the device)":
                                            round(ms_graph * 1e3, 2),
                                        "block-table fields from the caller": round(ms_ours * 1e3, 2),
                                        "mask kernel on gather_slots + mask": round(ms_masked * 1e3, 2)},
                   "kv_bytes_per_call": kv},
        "roofline": {"bound": "hbm", "achieved": round(kv / (ms_ref * 1e-3) / 1e9, 2), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(kv / (ms_ref * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4), "traffic": None,
                     "timed": "whole call (KV write + attention, eager launches, the step's check amortised)"},
        "cpu_baseline": None,
    }


def _measured_peak(bound: str, dtype: torch.dtype = torch.bfloat16) -> dict:
    """The roof the kernel is held against, measured on this device beside the
    published figure. HBM-bound kernels: a read-only stream of 4 GiB with the
    decode kernels' load form (``ir_hbm_read``: non-temporal 16-byte loads,
    ``value``) and a 1 GiB device-to-device copy (read + write bytes). MFMA-bound
    ones: an 8192^3 matmul of the kernel's dtype through torch's BLAS. Events
    around 10 runs after 3 warm-ups; the buffers exceed the 256 MB MALL."""
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
    x = torch.randn(n, n, device="cuda", dtype=dtype)
    y = torch.randn(n, n, device="cuda", dtype=dtype)
    name = "fp32" if dtype == torch.float32 else "bf16"
    return {"value": rate(lambda: x @ y, 2 * n**3 / 1e12), "unit": "TFLOP/s", "how": f"8192^3 {name} matmul (torch BLAS)"}


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
        line = {"prefill": _bench_prefill, "mixed": _bench_mixed, "rope": _bench_rope,
                "engine": _bench_engine, "reference-form": _bench_reference_form}[args.workload](args)
        line.update({"n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "timing": dict(_REPLAY_STATS)})
        print(json.dumps(line), flush=True)
        return 0
    from infrared_amd.workloads import make_decode_case

    args.config = args.config or "qwen7b-bf16"
    case = make_decode_case(args.config, "cuda", rotations=args.rotations, layout=args.layout)
    cfg = case.config
    kv = case.kv_bytes
    # bytes the kernel reads: with pairs, a shared prefix block once per pair
    read = case.unique_kv_bytes if args.pairs else kv
    info, eager_ms, graph_ms, kernel_ms, outs = _gpu_decode(case, args)
    us = graph_ms * 1e3
    gbps = kv / (graph_ms * 1e-3) / 1e9
    kgbps = read / (kernel_ms * 1e-3) / 1e9
    check = None
    if args.check:
        from oracle import naive as O

        ref = O.decode_reference(
            case.q.cpu(), case.k_cache.cpu(), case.v_cache.cpu(), case.block_tables[0].cpu(),
            case.context_lens.cpu(), cfg.block_size, cfg.scale,
        )
        check = round((outs[0].float().cpu() - ref).abs().max().item(), 6)
    scatter = _gpu_scatter(case, args) if args.mode == "graph" else None
    if args.copy_calib_mib > 0:
        _copy_calibration(args.copy_calib_mib)
    cpu = _cpu_baseline(case, args) if args.cpu_iters > 0 else None
    sched = ("pairs_" if args.pairs else "planned_") if info["schedule"] == "planned" else ""
    lay = "" if args.layout == "head_major" else f"{args.layout}_"
    traffic, traffic_src = _traffic(f"decode_{sched}{lay}{args.config}")
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
            "unique_kv_bytes_per_call": case.unique_kv_bytes,
            "rotations": args.rotations,
            "pool_layout": args.layout,
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
                      f" launches alone, {args.mode}, events on the launch stream"
                      + ("; achieved counts each shared prefix block once per pair" if args.pairs else "")),
        },
        "cpu_baseline": cpu,
        "scatter": scatter,
    }
    line["timing"] = dict(_REPLAY_STATS)
    if check is not None:
        line["max_abs_err_vs_fp32_oracle"] = check
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
