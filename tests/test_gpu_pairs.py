"""GPU parity of the planned decode with shared-prefix pairs
(``IR_PLAN_SHARE_GROUPS``): sequences b, b + 1 whose block tables begin with
the same block ids run as one unit per KV head, both sequences' query heads in
one MFMA tile, the shared blocks read once. Every output is still the
attention of its own sequence over its own keys, so the oracle is the
per-sequence decode reference (max-abs <= 1e-4 fp32, <= 2e-2 bf16/fp16 against
fp32); the plan's header records how many pairs it formed."""

from __future__ import annotations

import math

import pytest
import torch

from infrared_amd import kernels
from infrared_amd._lib import ERR_BLOCK_RANGE, ERR_PLAN
from infrared_amd.workloads import make_decode_case
from oracle import naive as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def _case(ctxs, shares, hq=28, hkv=4, d=128, dtype=torch.bfloat16, seed=0):
    """Sequences with contexts `ctxs`; each (i, j, n) of `shares` gives
    sequence j the first n block ids of sequence i's table."""
    gen = torch.Generator().manual_seed(seed)
    bs = 16
    nblk = [max(1, -(-c // bs)) for c in ctxs]
    pool = math.ceil(1.25 * sum(nblk)) + 4
    perm = torch.randperm(pool, generator=gen)
    bt = torch.zeros(len(ctxs), max(nblk), dtype=torch.int32)
    off = 0
    for i, n in enumerate(nblk):
        bt[i, :n] = perm[off:off + n].to(torch.int32)
        off += n
    for i, j, n in shares:
        bt[j, :n] = bt[i, :n]
    dgen = torch.Generator(device=DEV).manual_seed(seed)
    shape = (pool * bs, hkv, d)
    k = torch.randn(shape, generator=dgen, device=DEV).to(dtype).permute(1, 0, 2).contiguous().permute(1, 0, 2)
    v = torch.randn(shape, generator=dgen, device=DEV).to(dtype).permute(1, 0, 2).contiguous().permute(1, 0, 2)
    q = torch.randn(len(ctxs), hq, d, generator=dgen, device=DEV).to(dtype)
    return q, k, v, bt.to(DEV), torch.tensor(ctxs, dtype=torch.int32, device=DEV), pool


def _run(q, k, v, bt, cl, share, err=None, plan_buf=None):
    hq, d = q.shape[1], q.shape[2]
    scale = d**-0.5
    plan = kernels.decode_plan(bt, cl, hq, k, 16, buf=plan_buf, err_flags=err, share_groups=share)
    ctr = torch.zeros(kernels.decode_num_counters(q.shape[0], hq, k.shape[1]), dtype=torch.int32, device=DEV)
    ws = torch.full((kernels.planned_workspace_bytes(q.shape[0], hq, k.shape[1], d) // 4 + 64,), 2,
                    dtype=torch.int32, device=DEV).view(torch.uint8)
    out = kernels.paged_decode_planned(q, k, v, plan, scale, workspace=ws, err_flags=err, counters=ctr)
    return out, plan, ctr


def _pairs_in(plan) -> int:
    return int(plan.buf[:16].view(torch.int32)[3].item())


def _check(q, k, v, bt, cl, npairs, dtype=torch.bfloat16):
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    out, plan, ctr = _run(q, k, v, bt, cl, True, err)
    base, _, _ = _run(q, k, v, bt, cl, False)
    torch.cuda.synchronize()
    assert err.item() == 0
    assert int(ctr.abs().sum()) == 0
    assert _pairs_in(plan) == npairs
    ref = O.decode_reference(q.cpu(), k.cpu(), v.cpu(), bt.cpu(), cl.cpu(), 16, q.shape[2]**-0.5, torch.float32)
    diff = (out.float().cpu() - ref).abs().max().item()
    assert diff <= TOL[dtype], diff
    assert (out.float() - base.float()).abs().max().item() <= TOL[dtype]
    return out


def test_pairs_full_shape_parity():
    """The 64-sequence workload whose pairs (2i, 2i+1) share half the shorter
    context: 32 pairs, outputs within the bar of the oracle and of the
    unpaired plan on the same metadata."""
    case = make_decode_case("qwen7b-pairs", DEV)
    assert case.shared_tokens > 0
    _check(case.q, case.k_cache, case.v_cache, case.block_tables[0], case.context_lens, 32)


@pytest.mark.parametrize("ctxs,shares,npairs", [
    ([700, 900, 50, 2000], [(0, 1, 20)], 1),                    # one pair, the rest alone
    ([700, 900, 800, 300], [(0, 1, 30), (0, 2, 30)], 1),         # three share: (0, 1) pair, 2 alone
    ([100, 700, 900, 300], [(1, 2, 25)], 1),                     # a pair at an odd position
    ([48, 700, 33, 47], [(0, 1, 3), (2, 3, 2)], 2),               # first sequence wholly shared; 2 blocks of 33/47
    ([700, 48], [(0, 1, 3)], 1),                                  # second sequence wholly shared
    ([700, 900], [(0, 1, 1)], 1),                                 # one shared block
    ([15, 700, 12, 12], [(0, 1, 1), (2, 3, 1)], 0),               # no whole block inside both contexts
    ([900, 900, 900, 900], [(0, 1, 40), (1, 2, 40), (2, 3, 40)], 2),  # a run of four: (0, 1), (2, 3)
])
def test_pairs_shapes(ctxs, shares, npairs):
    q, k, v, bt, cl, _ = _case(ctxs, shares)
    _check(q, k, v, bt, cl, npairs)


def test_pairs_diverge_then_match_again():
    """The shared prefix ends at the first differing block even when a later
    block id matches again."""
    q, k, v, bt, cl, _ = _case([900, 900], [(0, 1, 20)])
    bt[1, 25] = bt[0, 25]
    _check(q, k, v, bt, cl, 1)


@pytest.mark.parametrize("hq,hkv,d,dtype,npairs", [
    (32, 4, 128, torch.bfloat16, 2),   # 8 query heads per KV head: a pair fills all 16 columns
    (36, 4, 128, torch.bfloat16, 0),   # 9 per KV head: a pair does not fit, the flag is ignored
    (14, 2, 64, torch.float16, 2),
    (14, 2, 64, torch.float32, 2),
])
def test_pairs_head_shapes(hq, hkv, d, dtype, npairs):
    q, k, v, bt, cl, _ = _case([700, 900, 400, 1300, 90], [(0, 1, 20), (2, 3, 10)], hq=hq, hkv=hkv, d=d,
                               dtype=dtype)
    _check(q, k, v, bt, cl, npairs, dtype)


def test_pairs_bad_block_in_shared_prefix():
    """A bad block id inside the shared prefix is flagged and its keys masked
    for both sequences, as the fixed-partition kernel does."""
    q, k, v, bt, cl, pool = _case([700, 900, 300], [(0, 1, 20)])
    bt[0, 5] = pool + 7
    bt[1, 5] = pool + 7
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    out, plan, _ = _run(q, k, v, bt, cl, True, err)
    fixed = kernels.paged_decode(q, k, v, bt, cl, 16, q.shape[2]**-0.5)
    torch.cuda.synchronize()
    assert err.item() & ERR_BLOCK_RANGE
    assert _pairs_in(plan) == 1
    assert (out.float() - fixed.float()).abs().max().item() <= 2 * TOL[torch.bfloat16]


def test_pairs_plan_run_without_the_flag_writes_nothing():
    """A plan that formed pairs, run by the kernel without pairs, flags
    IR_ERR_PLAN and leaves the output untouched."""
    q, k, v, bt, cl, _ = _case([700, 900, 300], [(0, 1, 20)])
    plan = kernels.decode_plan(bt, cl, q.shape[1], k, 16, share_groups=True)
    wrong = kernels.DecodePlan(**{**plan.__dict__, "share_groups": False})
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = torch.full_like(q, 3.0)
    kernels.paged_decode_planned(q, k, v, wrong, q.shape[2]**-0.5, out=out, err_flags=err)
    torch.cuda.synchronize()
    assert err.item() & ERR_PLAN
    assert bool((out == 3.0).all())


def test_pairs_graph_capture_replays():
    """Plan (with pairs) + two layers captured in one hipGraph: replays equal
    the eager calls bit for bit, with eager work between replays."""
    case = make_decode_case("qwen7b-pairs", DEV, num_seqs=16)
    bt, cl = case.block_tables[0], case.context_lens
    hq = case.config.num_q_heads
    d = case.config.head_dim
    plan_buf = torch.empty(kernels.decode_plan_bytes(16, hq, 4, bt.shape[1], 16), dtype=torch.uint8, device=DEV)
    ws = torch.empty(kernels.planned_workspace_bytes(16, hq, 4, d), dtype=torch.uint8, device=DEV)
    ctr = torch.zeros(kernels.decode_num_counters(16, hq, 4), dtype=torch.int32, device=DEV)
    q2 = torch.randn_like(case.q.float()).to(case.q.dtype)
    outs = [torch.empty_like(case.q), torch.empty_like(case.q)]

    def step():
        plan = kernels.decode_plan(bt, cl, hq, case.k_cache, 16, buf=plan_buf, share_groups=True)
        for i, qq in enumerate((case.q, q2)):
            kernels.paged_decode_planned(qq, case.k_cache, case.v_cache, plan, case.config.scale, out=outs[i],
                                         workspace=ws, counters=ctr)

    step()
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for _ in range(3):
        for o in outs:
            o.zero_()
        plan_buf.fill_(5)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(o, e) for o, e in zip(outs, eager))
    assert int(ctr.abs().sum()) == 0


def test_pairs_through_the_seam():
    """``paged_attention`` on a decode batch that fills the device, where the
    prefix cache gave consecutive sequences the same leading blocks: the step's
    plan forms the pairs, and every layer matches the oracle."""
    from infrared_amd import PagedKVPool, metadata, paged_attention

    bs, h_kv, n_rep, d, layers, b = 16, 4, 7, 128, 2, 80
    g = torch.Generator().manual_seed(31)
    num_cached = torch.randint(40, 900, (b,), generator=g).tolist()
    nblk = [metadata.blocks_for(nc + 1, bs) for nc in num_cached]
    perm = torch.randperm(sum(nblk) + 64, generator=g).tolist()
    tables, off = [], 0
    for nb in nblk:
        tables.append(perm[off:off + nb])
        off += nb
    for i in range(0, b - 1, 2):  # pairs share half of the shorter cached prefix
        sh = min(num_cached[i], num_cached[i + 1]) // 2 // bs
        tables[i + 1][:sh] = tables[i][:sh]
    pool = PagedKVPool(layers, len(perm), bs, h_kv, d, torch.bfloat16, device=DEV, strict=True)
    pool.k.normal_()
    pool.v.normal_()
    paged, mask = metadata.decode_context(pool, tables, num_cached)
    for layer in range(layers):
        q = torch.randn(b, 1, h_kv * n_rep, d, device=DEV).bfloat16()
        k = torch.randn(b, 1, h_kv, d, device=DEV).bfloat16()
        v = torch.randn(b, 1, h_kv, d, device=DEV).bfloat16()
        out = paged_attention(q, k, v, paged, mask, layer, d**-0.5, n_rep)
        assert paged.decode_plan is not None and paged.decode_plan.share_groups
        ref = O.paged_attention_naive(q.float().cpu(), pool.k[layer].float().cpu(), pool.v[layer].float().cpu(),
                                      paged.gather_slots.cpu(), mask.float().cpu(), d**-0.5, n_rep)
        assert (out.float().cpu() - ref).abs().max().item() <= 2e-2
    expect = sum(1 for i in range(0, b - 1, 2) if min(num_cached[i], num_cached[i + 1]) // 2 // bs > 0)
    assert _pairs_in(paged.decode_plan) == expect > 0
