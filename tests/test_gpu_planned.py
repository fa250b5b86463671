"""GPU parity of the planned (work-balanced) decode: ``ir_paged_decode_plan``
once per batch of decode metadata, ``ir_paged_decode_planned`` per layer,
called through the C ABI and checked against the CPU oracle on the same
seeded inputs (max-abs <= 1e-4 fp32, <= 2e-2 bf16/fp16 against fp32).

The cases are those of the fixed-partition decode tests -- the reference's
decode shapes, skewed long contexts, empty rows, a single 32k-token sequence,
wide batches, bad block ids -- plus what is new with a plan: one plan shared by
several layers and calls, slices that cut a sequence between workgroups (the
last-arriving workgroup merges; counters return to zero), and hipGraph capture
of plan + runs replayed with fresh metadata.
"""

from __future__ import annotations

import pytest
import torch

from infrared_amd import PagedContext, PagedKVPool, kernels, metadata, paged_attention
from infrared_amd._lib import ERR_BLOCK_RANGE, ERR_CONTEXT_RANGE
from infrared_amd.workloads import DecodeConfig, make_decode_case
from oracle import naive as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def _err():
    return torch.zeros(1, dtype=torch.int32, device=DEV)


def _garbage(nbytes: int) -> torch.Tensor:
    """Scratch workspace whose every int32 reads 2 (partial rows start as garbage)."""
    return torch.full(((nbytes + 3) // 4,), 2, dtype=torch.int32, device=DEV).view(torch.uint8)


def _run_planned(case, bt=None, cl=None, err=None, ws=None, q=None, plan=None, scale=None, ctr=None):
    cfg = case.config
    scale = cfg.scale if scale is None else scale
    bt = case.block_tables[0] if bt is None else bt
    cl = case.context_lens if cl is None else cl
    q = case.q if q is None else q
    if plan is None:
        plan = kernels.decode_plan(bt, cl, cfg.num_q_heads, case.k_cache, cfg.block_size, err_flags=err)
    if ws is None:
        ws = _garbage(kernels.planned_workspace_bytes(cfg.num_seqs, cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim))
    if ctr is None:
        ctr = torch.zeros(kernels.decode_num_counters(cfg.num_seqs, cfg.num_q_heads, cfg.num_kv_heads),
                          dtype=torch.int32, device=DEV)
    out = kernels.paged_decode_planned(q, case.k_cache, case.v_cache, plan, scale, workspace=ws, err_flags=err,
                                       counters=ctr)
    return out, plan, ctr


def _check_planned(case, bt=None, cl=None):
    cfg = case.config
    bt = case.block_tables[0] if bt is None else bt
    cl = case.context_lens if cl is None else cl
    err = _err()
    out, _, ctr = _run_planned(case, bt, cl, err)
    torch.cuda.synchronize()
    assert err.item() == 0
    assert int(ctr.abs().sum()) == 0
    ref = O.decode_reference(case.q.cpu(), case.k_cache.cpu(), case.v_cache.cpu(), bt.cpu(), cl.cpu(),
                             cfg.block_size, cfg.scale, torch.float32)
    diff = (out.float().cpu() - ref).abs().max().item()
    assert diff <= TOL[cfg.dtype], f"{cfg.name}: max-abs {diff}"
    return out


@pytest.mark.parametrize("layout", ["head_major", "slot_major"])
def test_planned_qwen05b_fp32_parity(layout):
    """Qwen2.5-0.5B shape, fp32: 8 seqs, 14/2 heads, D=64, ctx U[1,512]; bar 1e-4."""
    _check_planned(make_decode_case("qwen0.5b-fp32", DEV, layout=layout))


@pytest.mark.parametrize("layout", ["head_major", "slot_major"])
def test_planned_qwen7b_bf16_full_size_parity(layout):
    """Qwen2.5-7B shape, bf16, 64 seqs with ctx U[512,4096]: nearly every slice
    cuts a sequence, so most outputs come from cross-workgroup merges."""
    _check_planned(make_decode_case("qwen7b-bf16", DEV, layout=layout))


def test_planned_skewed_long_context():
    """Lognormal contexts up to 32k: the longest sequence spans dozens of slices."""
    case = make_decode_case("qwen7b-skewed", DEV)
    assert int(case.context_lens.max()) > 4096
    _check_planned(case)


_SWEEP = [
    # (dtype, h_q, h_kv, d, bs)
    (torch.float32, 14, 2, 64, 16),
    (torch.float32, 8, 8, 128, 16),
    (torch.bfloat16, 28, 4, 128, 32),
    (torch.bfloat16, 16, 2, 128, 16),
    (torch.bfloat16, 40, 2, 64, 16),   # two head groups per KV head
    (torch.bfloat16, 64, 2, 128, 16),  # two full head groups
    (torch.float16, 28, 4, 128, 16),
    (torch.float16, 12, 2, 64, 32),
]


@pytest.mark.parametrize("dtype,h_q,h_kv,d,bs", _SWEEP)
def test_planned_shape_sweep(dtype, h_q, h_kv, d, bs):
    """GQA groups 1..32, both head dims, block sizes 16 and 32, and context
    lengths on both sides of tile and block boundaries."""
    cfg = DecodeConfig(f"psweep-{h_q}-{h_kv}-{d}-{bs}", 7, h_q, h_kv, d, bs, dtype, "uniform", 300, 300, seed=h_q + bs)
    case = make_decode_case(cfg, DEV)
    case.context_lens.copy_(torch.tensor([1, 15, 16, 17, 31, 33, 300], dtype=torch.int32))
    _check_planned(case)


_MIX_CFG = DecodeConfig("mixed-lengths", 8, 28, 4, 128, 16, torch.bfloat16, "uniform", 5000, 5000, seed=11)


def test_planned_mixed_lengths_with_empty_rows():
    """Empty rows (zero output, written once by the plan's list), one-token rows
    and long ones in one batch."""
    case = make_decode_case(_MIX_CFG, DEV)
    case.context_lens.copy_(torch.tensor([0, 1, 5000, 0, 17, 4096, 0, 2048], dtype=torch.int32))
    out = _check_planned(case)
    for r in (0, 3, 6):
        assert out[r].float().abs().max().item() == 0.0


@pytest.mark.parametrize("ctx", [1, 16, 32768])
def test_planned_single_sequence(ctx):
    """One sequence: one key (a single busy workgroup), one tile, and 32k keys
    (every CU takes a slice of each of the 4 units; 64-way merges)."""
    cfg = DecodeConfig(f"p-one-seq-{ctx}", 1, 28, 4, 128, 16, torch.bfloat16, "uniform", ctx, ctx, seed=ctx)
    _check_planned(make_decode_case(cfg, DEV))


@pytest.mark.parametrize("num_seqs", [600, 1024])
def test_planned_wide_batches(num_seqs):
    """Many short rows (several units per slice) up to the 1024-sequence limit."""
    cfg = DecodeConfig(f"p-batch-{num_seqs}", num_seqs, 8, 2, 64, 16, torch.float16, "uniform", 1, 64, seed=5)
    _check_planned(make_decode_case(cfg, DEV))


def test_planned_all_rows_empty():
    case = make_decode_case(_MIX_CFG, DEV)
    case.context_lens.zero_()
    out = _check_planned(case)
    assert out.float().abs().max().item() == 0.0


def test_planned_plan_shared_by_layers_and_calls():
    """One plan serves three layers (different q and pool layers, same strides)
    on a shared workspace whose partial rows start as garbage; every call
    matches the oracle, repeats bit for bit, and leaves the counters at zero."""
    cfg = DecodeConfig("p-layers", 16, 28, 4, 128, 16, torch.bfloat16, "uniform", 64, 3000, seed=21)
    case = make_decode_case(cfg, DEV)
    bt, cl = case.block_tables[0], case.context_lens
    pool_k = torch.randn(3, *case.k_cache.shape, device=DEV).to(cfg.dtype)
    pool_v = torch.randn(3, *case.v_cache.shape, device=DEV).to(cfg.dtype)
    plan = kernels.decode_plan(bt, cl, cfg.num_q_heads, pool_k[0], 16)
    ws = _garbage(kernels.planned_workspace_bytes(16, 28, 4, 128))
    ctr = torch.zeros(kernels.decode_num_counters(16, 28, 4), dtype=torch.int32, device=DEV)
    for layer in range(3):
        q = torch.randn_like(case.q)
        outs = [kernels.paged_decode_planned(q, pool_k[layer], pool_v[layer], plan, cfg.scale, workspace=ws,
                                             counters=ctr) for _ in range(2)]
        torch.cuda.synchronize()
        assert torch.equal(outs[0], outs[1])
        assert int(ctr.abs().sum()) == 0
        ref = O.decode_reference(q.cpu(), pool_k[layer].cpu(), pool_v[layer].cpu(), bt.cpu(), cl.cpu(), 16, cfg.scale)
        assert (outs[0].float().cpu() - ref).abs().max().item() <= TOL[cfg.dtype]


def test_planned_calls_of_different_batch_sizes_share_scratch_and_counters():
    """Batches of 128, 109 and 128 sequences in turn on one scratch workspace
    and one counters buffer (an engine's steps through one pool): a smaller
    call's partial rows never land on a larger call's counters, every call
    matches the oracle and the counters return to zero."""
    cfg = DecodeConfig("p-shapes", 128, 28, 4, 128, 16, torch.bfloat16, "uniform", 1, 600, seed=31)
    case = make_decode_case(cfg, DEV)
    ws = _garbage(kernels.planned_workspace_bytes(128, 28, 4, 128))
    ctr = torch.zeros(kernels.decode_num_counters(128, 28, 4), dtype=torch.int32, device=DEV)
    for b in (128, 109, 128, 109):
        bt, cl, q = case.block_tables[0][:b], case.context_lens[:b], case.q[:b]
        plan = kernels.decode_plan(bt, cl, 28, case.k_cache, 16)
        out = kernels.paged_decode_planned(q, case.k_cache, case.v_cache, plan, cfg.scale, workspace=ws, counters=ctr)
        torch.cuda.synchronize()
        assert int(ctr.abs().sum()) == 0
        ref = O.decode_reference(q.cpu(), case.k_cache.cpu(), case.v_cache.cpu(), bt.cpu(), cl.cpu(), 16, cfg.scale)
        assert (out.float().cpu() - ref).abs().max().item() <= TOL[cfg.dtype], f"batch {b}"


def test_planned_flags_bad_block_ids_and_contexts():
    """Out-of-pool block ids and over-long contexts are flagged by the plan and
    their keys masked (never read), as in the fixed-partition kernel."""
    case = make_decode_case("qwen7b-bf16", DEV, num_seqs=4)
    bt = case.block_tables[0].clone()
    bt[1, 3] = case.pool_blocks + 100
    err = _err()
    got, _, _ = _run_planned(case, bt=bt, err=err)
    fixed = kernels.paged_decode(case.q, case.k_cache, case.v_cache, bt, case.context_lens, 16, case.config.scale)
    torch.cuda.synchronize()
    assert err.item() & ERR_BLOCK_RANGE
    assert (got.float() - fixed.float()).abs().max().item() <= 2 * TOL[torch.bfloat16]
    cl = case.context_lens.clone()
    cl[0] = bt.shape[1] * 16 + 50
    err.zero_()
    _run_planned(case, cl=cl, err=err)
    torch.cuda.synchronize()
    assert err.item() & ERR_CONTEXT_RANGE


def test_planned_one_hot_probe_returns_exact_v_row():
    """A key whose score dwarfs the rest makes the output equal its V row: pins
    the plan's per-tile pool offsets (block id, offset in block, KV head)
    exactly, through a cross-workgroup merge where the key's slice is not the
    last to arrive."""
    case = make_decode_case("qwen7b-bf16", DEV, num_seqs=3)
    bt = case.block_tables[0]
    for i in range(3):
        n = int(case.context_lens[i])
        p = n // 2 + 3
        s = int(bt[i, p // 16]) * 16 + p % 16
        for g in range(4):
            case.k_cache[s, g] = (case.q[i, 7 * g] * 64).to(case.k_cache.dtype)
            for h in range(7 * g, 7 * g + 7):
                case.q[i, h] = case.q[i, 7 * g]
    out, _, _ = _run_planned(case, scale=1.0)
    torch.cuda.synchronize()
    for i in range(3):
        n = int(case.context_lens[i])
        p = n // 2 + 3
        s = int(bt[i, p // 16]) * 16 + p % 16
        for h in range(28):
            assert torch.equal(out[i, h], case.v_cache[s, h // 7]), (i, h)


def test_planned_graph_capture_replays_with_fresh_metadata():
    """Plan + two layers captured in one hipGraph; replays after new context
    lengths are copied into the captured buffers match eager calls bit for bit,
    with eager work and synchronisations between the replays."""
    cfg = DecodeConfig("p-graph", 12, 28, 4, 128, 16, torch.bfloat16, "uniform", 2000, 2000, seed=9)
    case = make_decode_case(cfg, DEV)
    bt = case.block_tables[0].clone()
    cl = case.context_lens.clone()
    q2 = torch.randn(2, *case.q.shape, device=DEV).to(cfg.dtype)
    plan_buf = torch.empty(kernels.decode_plan_bytes(12, 28, 4, bt.shape[1], 16), dtype=torch.uint8, device=DEV)
    ws = _garbage(kernels.planned_workspace_bytes(12, 28, 4, 128))
    ctr = torch.zeros(kernels.decode_num_counters(12, 28, 4), dtype=torch.int32, device=DEV)
    outs = torch.empty(2, *case.q.shape, dtype=cfg.dtype, device=DEV)

    def step():
        plan = kernels.decode_plan(bt, cl, 28, case.k_cache, 16, buf=plan_buf)
        for layer in range(2):
            kernels.paged_decode_planned(q2[layer], case.k_cache, case.v_cache, plan, cfg.scale, out=outs[layer],
                                         workspace=ws, counters=ctr)

    step()  # warm-up outside capture
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            step()
    torch.cuda.current_stream().wait_stream(stream)
    g = torch.Generator().manual_seed(4)
    for it in range(4):
        cl.copy_(torch.randint(1, 2001, (12,), generator=g).to(torch.int32))
        graph.replay()
        torch.cuda.synchronize()
        got = outs.clone()
        plan = kernels.decode_plan(bt, cl, 28, case.k_cache, 16)
        want = [kernels.paged_decode_planned(q2[layer], case.k_cache, case.v_cache, plan, cfg.scale) for layer in range(2)]
        torch.cuda.synchronize()
        for layer in range(2):
            assert torch.equal(got[layer], want[layer]), f"replay {it} layer {layer}"
        assert int(ctr.abs().sum()) == 0


def test_plannable_shapes_and_rejections():
    """Batches beyond 1024 or block sizes not a multiple of 16 are not planned
    (the seam keeps the fixed-partition kernel for them); a plan refuses a pool
    or query that differs from the one it was built for."""
    assert kernels.decode_plan_bytes(1025, 28, 4, 16, 16) == 0
    assert kernels.decode_plan_bytes(8, 28, 4, 16, 8) == 0
    assert kernels.decode_plan_bytes(8, 28, 4, 16, 16) > 0
    case = make_decode_case("qwen7b-bf16", DEV, num_seqs=4)
    plan = kernels.decode_plan(case.block_tables[0], case.context_lens, 28, case.k_cache, 16)
    with pytest.raises(RuntimeError):
        kernels.paged_decode_planned(case.q[:3], case.k_cache, case.v_cache, plan, 0.1)
    other = case.k_cache.contiguous()  # slot-major strides instead of head-major
    with pytest.raises(RuntimeError):
        kernels.paged_decode_planned(case.q, other, other, plan, 0.1)


def test_seam_decode_builds_the_plan_once_per_context():
    """Through ``paged_attention``: a batch with a unit per CU takes the planned
    schedule -- the first decode layer of a context builds its plan, later
    layers reuse it -- and every layer matches the oracle; a small batch keeps
    the fixed-partition kernel (no plan)."""
    bs, h_kv, n_rep, d, layers = 16, 4, 7, 128, 3
    for b, planned in ((80, True), (12, False)):
        g = torch.Generator().manual_seed(13 + b)
        num_cached = torch.randint(0, 700, (b,), generator=g).tolist()
        nblk = [metadata.blocks_for(nc + 1, bs) for nc in num_cached]
        perm = torch.randperm(sum(nblk) + 64, generator=g).tolist()
        tables, off = [], 0
        for nb in nblk:
            tables.append(perm[off : off + nb])
            off += nb
        pool = PagedKVPool(layers, len(perm), bs, h_kv, d, torch.bfloat16, device=DEV, strict=True)
        pool.k.normal_()
        pool.v.normal_()
        paged, mask = metadata.decode_context(pool, tables, num_cached)
        assert isinstance(paged, PagedContext) and paged.decode_plan is None
        assert kernels.decode_plan_pays(b, h_kv * n_rep, h_kv, paged.block_tables.shape[1], bs) == planned
        plans = []
        for layer in range(layers):
            q = torch.randn(b, 1, h_kv * n_rep, d, device=DEV).bfloat16()
            k = torch.randn(b, 1, h_kv, d, device=DEV).bfloat16()
            v = torch.randn(b, 1, h_kv, d, device=DEV).bfloat16()
            out = paged_attention(q, k, v, paged, mask, layer, d**-0.5, n_rep)
            plans.append(paged.decode_plan)
            ref = O.paged_attention_naive(q.float().cpu(), pool.k[layer].float().cpu(), pool.v[layer].float().cpu(),
                                          paged.gather_slots.cpu(), mask.float().cpu(), d**-0.5, n_rep)
            assert (out.float().cpu() - ref).abs().max().item() <= 2e-2
        if planned:
            assert plans[0] is not None and all(p is plans[0] for p in plans)
        else:
            assert all(p is None for p in plans)


def test_seam_graph_decoder_replays_the_planned_step():
    """HipGraphDecoder over a batch that fills the device (bucket 128 x 4 KV
    heads): the captured step holds the plan build and two planned layers;
    replays with new contexts equal the eager step at the same bucket bit for
    bit and the tight (unpadded) eager step within the bf16 bar."""
    from infrared_amd.hip_graph import HipGraphDecoder, build_decode_static_inputs, pick_bucket

    bs, h_kv, n_rep, d, layers = 16, 4, 7, 128, 2
    dtype = torch.bfloat16
    pool = PagedKVPool(layers, 128 * 40, bs, h_kv, d, dtype, device=DEV)
    pool.k.normal_()
    pool.v.normal_()
    gen = torch.Generator(device=DEV).manual_seed(5)
    qkv = torch.randn(layers, 128, 1, h_kv * (n_rep + 2), d, generator=gen, device=DEV).to(dtype)

    def step(buf, paged):
        outs = []
        ids = buf.ids[:, 0]
        for layer in range(layers):
            x = qkv[layer].index_select(0, ids)
            q = x[:, :, : h_kv * n_rep].contiguous()
            k = x[:, :, h_kv * n_rep : h_kv * (n_rep + 1)].contiguous()
            v = x[:, :, h_kv * (n_rep + 1) :].contiguous()
            outs.append(paged_attention(q, k, v, paged, buf.mask, layer, d**-0.5, n_rep))
        return torch.stack(outs, dim=1)

    dec = HipGraphDecoder(None, pool, max_num_seqs=128, t_max=640, block_size=bs, step_fn=step)
    tables = [list(range(i * 40, i * 40 + 40)) for i in range(128)]
    g = torch.Generator().manual_seed(6)
    for it in range(3):
        b = 100 + 9 * it
        num_cached = torch.randint(0, 600, (b,), generator=g).tolist()
        got = dec.decode(tables[:b], num_cached, list(range(b))).clone()
        bucket = pick_bucket(b, dec.buckets)
        assert bucket == 128 and kernels.decode_plan_pays(bucket, h_kv * n_rep, h_kv, 40, bs)
        outs = []
        for rows in (bucket, b):
            inp = build_decode_static_inputs(tables[:b], num_cached, list(range(b)), rows, 640, bs, DEV, dtype)
            paged = PagedContext(pool, inp.write_slots, inp.gather_slots, True, inp.block_tables, inp.context_lens)
            outs.append(step(inp, paged)[:b])
        torch.cuda.synchronize()
        assert torch.equal(got, outs[0]), f"replay {it} differs from eager at bucket {bucket}"
        assert (got.float() - outs[1].float()).abs().max().item() <= 2e-2, f"replay {it}: padded vs tight"
