"""The drop-in seam on the GPU: ``paged_attention`` with the reference's call
signature (both the block-table path and the gather_slots+mask path), the
pool's write/gather surface, and hipGraph capture/replay of a decode step."""

from __future__ import annotations

from dataclasses import dataclass

import pytest
import torch

from infrared_amd import PagedContext, PagedKVPool, kernels, metadata, paged_attention
from infrared_amd._lib import stream_ptr
from infrared_amd.hip_graph import HipGraphDecoder, build_decode_static_inputs, pick_bucket
from oracle import naive as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_reference_style_single_block_pool():
    """The reference's own GPU parity case (tests/test_triton_attention.py:155-187):
    b=2, sq=4, 2 kv heads, n_rep=2, d=64, causal mask over this step's tokens."""
    b, sq, h_kv, n_rep, d = 2, 4, 2, 2, 64
    torch.manual_seed(0)
    q = torch.randn(b, sq, h_kv * n_rep, d, device=DEV)
    k = torch.randn(b, sq, h_kv, d, device=DEV)
    v = torch.randn(b, sq, h_kv, d, device=DEV)
    allowed = torch.arange(sq, device=DEV)[None, :] <= torch.arange(sq, device=DEV)[:, None]
    mask = torch.zeros(b, 1, sq, sq, device=DEV).masked_fill(~allowed[None, None], torch.finfo(torch.float32).min)
    n = b * sq
    pool = PagedKVPool(1, 1, n, h_kv, d, torch.float32, device=DEV, strict=True)
    ctx = PagedContext(pool, torch.arange(n, device=DEV), torch.arange(n, device=DEV).reshape(b, sq))
    got = paged_attention(q, k, v, ctx, mask, 0, d**-0.5, n_rep)
    want = O.masked_attention(
        q.cpu(), O.repeat_kv(k.cpu(), n_rep), O.repeat_kv(v.cpu(), n_rep), mask.cpu(), d**-0.5
    )
    assert (got.cpu() - want).abs().max().item() <= 1e-4


@pytest.mark.parametrize("use_triton", [True, False])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_step_through_seam(use_triton, dtype):
    """One batched decode step as the engine issues it (infrared/engine/paged_engine.py:290-332):
    scatter the new K/V, then attend; the block-table path and the mask path both
    match the oracle run on the same pool."""
    g = torch.Generator().manual_seed(7)
    bs, h_kv, n_rep, d, b = 16, 4, 7, 128, 9
    num_cached = torch.randint(0, 900, (b,), generator=g).tolist()
    perm = torch.randperm(600, generator=g).tolist()
    tables, off = [], 0
    for nc in num_cached:
        nb = metadata.blocks_for(nc + 1, bs)
        tables.append(perm[off : off + nb])
        off += nb
    pool = PagedKVPool(2, 600, bs, h_kv, d, dtype, device=DEV, strict=True)
    pool.k.normal_()
    pool.v.normal_()
    paged, mask = metadata.decode_context(pool, tables, num_cached, use_triton=use_triton)
    q = torch.randn(b, 1, h_kv * n_rep, d, device=DEV).to(dtype)
    k = torch.randn(b, 1, h_kv, d, device=DEV).to(dtype)
    v = torch.randn(b, 1, h_kv, d, device=DEV).to(dtype)
    k_ref, v_ref = pool.k[1].cpu().clone(), pool.v[1].cpu().clone()
    out = paged_attention(q, k, v, paged, mask, 1, d**-0.5, n_rep)
    O.pool_write(k_ref, v_ref, k.reshape(-1, h_kv, d).cpu(), v.reshape(-1, h_kv, d).cpu(), paged.write_slots.cpu())
    assert torch.equal(pool.k[1].cpu(), k_ref) and torch.equal(pool.v[1].cpu(), v_ref)
    ref = O.paged_attention_naive(
        q.float().cpu(), k_ref.float(), v_ref.float(), paged.gather_slots.cpu(), mask.float().cpu(), d**-0.5, n_rep
    )
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    assert (out.float().cpu() - ref).abs().max().item() <= tol


@pytest.mark.parametrize("use_triton", [True, False])
def test_packed_prefill_and_decode_step_through_seam(use_triton):
    """A mixed step as the engine packs it (infrared/engine/paged_engine.py:461-516):
    two prefill chunks (one after a cached prefix) and three decode rows in one
    B=1 frame. The block-table path (prefill MFMA kernel) and the reference's
    gather_slots + varlen-mask path both match the oracle on the same pool."""
    g = torch.Generator().manual_seed(8)
    bs, h_kv, n_rep, d = 16, 4, 7, 128
    num_cached = [0, 300, 41, 1000, 7]
    q_lens = [77, 130, 1, 1, 1]
    perm = torch.randperm(400, generator=g).tolist()
    tables, off = [], 0
    for nc, n in zip(num_cached, q_lens):
        nb = metadata.blocks_for(nc + n, bs)
        tables.append(perm[off : off + nb])
        off += nb
    pool = PagedKVPool(1, 400, bs, h_kv, d, torch.bfloat16, device=DEV, strict=True)
    pool.k.normal_()
    pool.v.normal_()
    paged, mask = metadata.prefill_context(pool, tables, num_cached, q_lens, use_triton=use_triton, with_mask=True)
    total = sum(q_lens)
    q = torch.randn(1, total, h_kv * n_rep, d, device=DEV).to(torch.bfloat16)
    k = torch.randn(1, total, h_kv, d, device=DEV).to(torch.bfloat16)
    v = torch.randn(1, total, h_kv, d, device=DEV).to(torch.bfloat16)
    out = paged_attention(q, k, v, paged, mask, 0, d**-0.5, n_rep)
    bt = metadata.block_tables_tensor(tables, "cpu")
    ref = O.prefill_reference(q[0].cpu(), pool.k[0].cpu(), pool.v[0].cpu(), bt, paged.cu_seqlens_q.cpu(),
                              num_cached, bs, d**-0.5)
    assert (out[0].float().cpu() - ref).abs().max().item() <= 2e-2


@pytest.mark.parametrize("case", ["many-workgroups", "few-long"])
def test_prefill_step_builds_its_work_plan_once(case):
    """A prefill step whose workgroups outnumber the CUs, or one of few
    workgroups over a long context (one 200-token chunk after 3,000 cached: 48
    workgroups, items worth cutting): the first layer builds the work plan and
    caches it on the context, the second reuses it, and both layers' outputs
    equal the unplanned kernel (within the fp32 rounding of a cut item's merge)
    and match the oracle."""
    g = torch.Generator().manual_seed(9)
    bs, h_kv, n_rep, d = 16, 4, 7, 128
    if case == "many-workgroups":
        num_cached = [0, 2000, 160, 3000, 40, 40, 900, 1200]
        q_lens = [300, 300, 280, 300, 64, 300, 2, 250]
        assert kernels.prefill_plan_pays(len(q_lens), max(q_lens), h_kv * n_rep, h_kv, DEV)
    else:
        num_cached, q_lens = [3000], [200]
        assert not kernels.prefill_plan_pays(1, 200, h_kv * n_rep, h_kv, DEV)
        assert kernels.prefill_plan_pays(1, 200, h_kv * n_rep, h_kv, DEV, max_keys=3200)
        # fp32 items are 9 tokens, two workgroups resident per CU: 4 x 256
        # tokens (464 workgroups) start at once, 8 x 256 do not
        cus = torch.cuda.get_device_properties(DEV).multi_processor_count
        for nseq in (4, 8):
            wgs = nseq * -(-256 // 9) * h_kv
            assert kernels.prefill_plan_pays(nseq, 256, h_kv * n_rep, h_kv, DEV, dtype=torch.float32) == (
                wgs > 2 * cus)
    nblk = sum(metadata.blocks_for(c + n, bs) for c, n in zip(num_cached, q_lens))
    perm = torch.randperm(nblk + 10, generator=g).tolist()
    tables, off = [], 0
    for nc, n in zip(num_cached, q_lens):
        nb = metadata.blocks_for(nc + n, bs)
        tables.append(perm[off : off + nb])
        off += nb
    pool = PagedKVPool(2, nblk + 10, bs, h_kv, d, torch.bfloat16, device=DEV, strict=True)
    pool.k.normal_()
    pool.v.normal_()
    paged, _ = metadata.prefill_context(pool, tables, num_cached, q_lens)
    assert paged.prefill_plan is None
    total = sum(q_lens)
    for layer in range(2):
        q = torch.randn(1, total, h_kv * n_rep, d, device=DEV).to(torch.bfloat16)
        k = torch.randn(1, total, h_kv, d, device=DEV).to(torch.bfloat16)
        v = torch.randn(1, total, h_kv, d, device=DEV).to(torch.bfloat16)
        out = paged_attention(q, k, v, paged, None, layer, d**-0.5, n_rep)
        if layer == 0:
            plan = paged.prefill_plan
            assert plan is not None
        assert paged.prefill_plan is plan
        plain = kernels.paged_prefill(q[0], pool.k[layer], pool.v[layer], paged.block_tables, paged.cu_seqlens_q,
                                      paged.q_start, paged.max_q_len, bs, d**-0.5)
        assert (out[0].float() - plain.float()).abs().max().item() <= 2e-2
        bt = metadata.block_tables_tensor(tables, "cpu")
        ref = O.prefill_reference(q[0].cpu(), pool.k[layer].cpu(), pool.v[layer].cpu(), bt,
                                  paged.cu_seqlens_q.cpu(), num_cached, bs, d**-0.5)
        assert (out[0].float().cpu() - ref).abs().max().item() <= 2e-2


@pytest.mark.parametrize("layout", ["head_major", "slot_major"])
def test_pool_direct_slot_writes_feed_the_kernels(layout):
    """Reference callers write history straight into ``pool.k[layer, a:b]``
    (tests/test_cuda_graph.py:199-203); the kernels read it back in both layouts."""
    bs, h_kv, d = 8, 2, 64
    pool = PagedKVPool(2, 4, bs, h_kv, d, torch.float32, device=DEV, layout=layout)
    assert pool.k.shape == (2, 32, h_kv, d)
    k0 = torch.randn(3, h_kv, d, device=DEV)
    k1 = torch.randn(5, h_kv, d, device=DEV)
    pool.k[1, 0:3] = k0
    pool.v[1, 0:3] = k0 * 2
    pool.k[1, 8:13] = k1
    pool.v[1, 8:13] = k1 * 2
    k, v = pool.gather(1, torch.tensor([[0, 1, 2, 8, 9]], device=DEV))
    assert torch.equal(k[0, :3], k0) and torch.equal(k[0, 3:], k1[:2]) and torch.equal(v[0, :3], k0 * 2)
    bt = torch.tensor([[0], [1]], dtype=torch.int32, device=DEV)
    cl = torch.tensor([3, 5], dtype=torch.int32, device=DEV)
    gk, gv = pool.gather_blocks(1, bt, cl, 6)
    assert torch.equal(gk[0, :3], k0) and torch.equal(gk[1, :5], k1) and gk[0, 3:].eq(0).all()


def test_pool_gather_matches_indexing_and_strict_raises():
    pool = PagedKVPool(2, 8, 4, 2, 64, torch.bfloat16, device=DEV, strict=True)
    pool.k.normal_()
    pool.v.normal_()
    gs = torch.randint(0, 32, (3, 5), device=DEV)
    k, v = pool.gather(1, gs)
    assert torch.equal(k, pool.k[1][gs]) and torch.equal(v, pool.v[1][gs])
    with pytest.raises(IndexError, match="slot"):
        pool.write(0, torch.zeros(1, 2, 64, device=DEV, dtype=torch.bfloat16),
                   torch.zeros(1, 2, 64, device=DEV, dtype=torch.bfloat16),
                   torch.tensor([32], device=DEV))


def test_hip_graph_decode_replay_matches_eager():
    """Capture a 3-layer decode step (scatter + attention per layer) per bucket and
    replay it across growing contexts: every replay equals the eager step on the
    same bucket-padded inputs bit for bit, and its real rows match the tight
    (unpadded) eager step within the bf16 bar -- the padded-vs-tight gate of
    tests/test_cuda_graph.py:178-210, which the reference checks with allclose
    (the split-KV partition may differ between batch sizes)."""
    bs, h_kv, n_rep, d, layers = 16, 4, 7, 128, 3
    dtype = torch.bfloat16
    pool = PagedKVPool(layers, 512, bs, h_kv, d, dtype, device=DEV)
    pool.k.normal_()
    pool.v.normal_()
    gen = torch.Generator(device=DEV).manual_seed(3)
    qkv = torch.randn(layers, 8, 1, h_kv * (n_rep + 2), d, generator=gen, device=DEV).to(dtype)

    def step(buf, paged):
        # K/V are a function of the token id, so pad-by-repeat rows write the
        # same rows to the same slots, as a real model's would
        outs = []
        ids = buf.ids[:, 0]
        for layer in range(layers):
            x = qkv[layer].index_select(0, ids)
            q = x[:, :, : h_kv * n_rep].contiguous()
            k = x[:, :, h_kv * n_rep : h_kv * (n_rep + 1)].contiguous()
            v = x[:, :, h_kv * (n_rep + 1) :].contiguous()
            outs.append(paged_attention(q, k, v, paged, buf.mask, layer, d**-0.5, n_rep))
        return torch.stack(outs, dim=1)  # [B, layers, 1, H, D]

    dec = HipGraphDecoder(None, pool, max_num_seqs=8, t_max=1024, block_size=bs, step_fn=step)
    tables = [list(range(i * 64, i * 64 + 64)) for i in range(6)]
    for it, num_cached in enumerate([[5, 100, 300], [6, 101, 301], [17, 700, 2, 40, 900]]):
        b = len(num_cached)
        got = dec.decode(tables[:b], num_cached, list(range(b))).clone()
        bucket = pick_bucket(b, dec.buckets)
        outs = []
        for rows in (bucket, b):
            inp = build_decode_static_inputs(
                tables[:b], num_cached, list(range(b)), rows, 1024, bs, DEV, dtype
            )
            paged = PagedContext(pool, inp.write_slots, inp.gather_slots, True, inp.block_tables, inp.context_lens)
            outs.append(step(inp, paged)[:b])
        torch.cuda.synchronize()
        assert torch.equal(got, outs[0]), f"replay {it} differs from eager at bucket {bucket}"
        assert (got.float() - outs[1].float()).abs().max().item() <= 2e-2, f"replay {it}: padded vs tight"


def test_hip_graph_smaller_bucket_after_buffer_growth():
    """A bucket captured first keeps replaying correctly after a larger bucket's
    warm-up has grown (replaced) the pool's workspace, counters and plan
    buffer: the first graph still addresses the buffers it was captured with.
    The freed sizes are then handed out again, filled with ones (a counter
    read from them would skip merges), before the small bucket replays."""
    bs, h_kv, n_rep, d, layers, t_max = 16, 4, 7, 128, 2, 4096
    dtype = torch.bfloat16
    nblk = t_max // bs
    pool = PagedKVPool(layers, 64 * nblk, bs, h_kv, d, dtype, device=DEV)
    pool.k.normal_()
    pool.v.normal_()
    gen = torch.Generator(device=DEV).manual_seed(5)
    qkv = torch.randn(layers, 64, 1, h_kv * (n_rep + 2), d, generator=gen, device=DEV).to(dtype)

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

    dec = HipGraphDecoder(None, pool, max_num_seqs=64, t_max=t_max, block_size=bs, step_fn=step)
    tables = [list(range(i * nblk, (i + 1) * nblk)) for i in range(64)]
    rng = torch.Generator().manual_seed(11)

    def eager(b, num_cached):
        bucket = pick_bucket(b, dec.buckets)
        inp = build_decode_static_inputs(tables[:b], num_cached, list(range(b)), bucket, t_max, bs, DEV, dtype)
        paged = PagedContext(pool, inp.write_slots, inp.gather_slots, True, inp.block_tables, inp.context_lens)
        return step(inp, paged)[:b]

    small = [int(x) for x in torch.randint(1000, 4000, (4,), generator=rng)]
    dec.decode(tables[:4], small, list(range(4)))
    sizes = [t.numel() for t in (pool._workspace, pool._counters, pool._plan_buf)]
    large = [int(x) for x in torch.randint(1000, 4000, (64,), generator=rng)]
    dec.decode(tables[:64], large, list(range(64)))
    assert [t.numel() for t in (pool._workspace, pool._counters, pool._plan_buf)] != sizes, "no buffer grew"
    filler = [torch.ones(n // 4 + 1, dtype=torch.int32, device=DEV) for n in sizes for _ in range(4)]
    for it in range(3):
        small = [c + 1 for c in small]
        got = dec.decode(tables[:4], small, list(range(4))).clone()
        ref = eager(4, small)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"bucket-4 replay {it} after growth differs from eager"
    assert all(int(f.min()) == 1 and int(f.max()) == 1 for f in filler), "a replay wrote into freed memory"


@dataclass(slots=True)
class _ReferenceContext:
    """The reference's own PagedContext shape (infrared/cache/paged_kv_cache.py:75-91):
    no block-table fields, no room for any."""

    pool: PagedKVPool
    write_slots: torch.Tensor
    gather_slots: torch.Tensor
    use_triton: bool = True


@pytest.mark.parametrize("num_seqs", [4, 64])  # fixed partitions / planned schedule
def test_reference_decode_metadata_runs_the_block_table_kernels(num_seqs):
    """Unchanged reference callers pass only gather_slots + the decode mask. Their
    decode form is recognised (once per step: later layers reuse the derived
    tables), and every layer equals the block-table context's output bit for
    bit -- the same kernels on the same tables -- and the oracle."""
    bs, h_kv, n_rep, d, layers = 16, 4, 7, 128, 3
    g = torch.Generator().manual_seed(12)
    num_cached = [int(x) for x in torch.randint(0, 1500, (num_seqs,), generator=g)]
    tables = [list(range(i * 96, i * 96 + 96)) for i in range(num_seqs)]
    pool = PagedKVPool(layers, num_seqs * 96, bs, h_kv, d, torch.bfloat16, device=DEV)
    pool.k.normal_()
    pool.v.normal_()
    ours, mask = metadata.decode_context(pool, tables, num_cached)
    ref = _ReferenceContext(pool, ours.write_slots, ours.gather_slots)
    dgen = torch.Generator(device=DEV).manual_seed(1)
    forms = []
    for layer in range(layers):
        q = torch.randn(num_seqs, 1, h_kv * n_rep, d, generator=dgen, device=DEV).bfloat16()
        k = torch.randn(num_seqs, 1, h_kv, d, generator=dgen, device=DEV).bfloat16()
        v = torch.randn(num_seqs, 1, h_kv, d, generator=dgen, device=DEV).bfloat16()
        got = paged_attention(q, k, v, ref, mask, layer, d**-0.5, n_rep)
        forms.append(pool._ref_form[1])
        want = paged_attention(q, k, v, ours, mask, layer, d**-0.5, n_rep)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"layer {layer}"
        assert (forms[-1].decode_plan is not None) == (num_seqs == 64)
        expect = O.decode_reference(q[:, 0].cpu(), pool.k[layer].cpu(), pool.v[layer].cpu(),
                                    ours.block_tables.cpu(), ours.context_lens.cpu(), bs, d**-0.5)
        assert (got[:, 0].float().cpu() - expect).abs().max().item() <= 2e-2
    assert forms[0] is not None and all(f is forms[0] for f in forms)
    assert forms[0].verdict() is True  # later layers ran the block-table kernels alone
    assert torch.equal(forms[0].context_lens, ours.context_lens)
    for i, c in enumerate(ours.context_lens.tolist()):  # (entries past a context are never read)
        n = -(-c // bs)
        assert torch.equal(forms[0].block_tables[i, :n], ours.block_tables[i, :n])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("num_blocks", [600, 2**28])  # slots divided in 32 bits / in 64 bits
def test_decode_form_check_over_mask_dtypes(dtype, num_blocks):
    """The decode-form check on every mask dtype: context lengths and block
    tables come back exact (contexts longer than one pass of a lane's loads
    included); a NaN, a masked value above -6e4, a hidden key inside a context,
    a slot off its block or a row with no visible key each reject the
    metadata, while -inf still masks. With IR_FORM_CLEAR_ON_FAIL a rejected
    check leaves every context length 0."""
    bs = 16
    g = torch.Generator().manual_seed(31)
    num_cached = [0, 4999, 17, 4096, 1]
    perm = torch.randperm(600, generator=g).tolist()
    tables, off = [], 0
    for nc in num_cached:
        nb = metadata.blocks_for(nc + 1, bs)
        tables.append(perm[off : off + nb])
        off += nb
    t = max(num_cached) + 1
    gs = torch.zeros(len(tables), t, dtype=torch.int64)
    mask = torch.full((len(tables), 1, 1, t), torch.finfo(dtype).min, dtype=dtype)
    for i, (bt, nc) in enumerate(zip(tables, num_cached)):
        gs[i, : nc + 1] = torch.tensor([O.slot(bt, p, bs) for p in range(nc + 1)])
        mask[i, 0, 0, : nc + 1] = 0
    ctx_want = [nc + 1 for nc in num_cached]

    record = torch.zeros(1, dtype=torch.int64, pin_memory=True)
    tags = iter(range(7, 100))

    def run(gs_, mask_):
        tag = next(tags)
        bt, ctx, bad = kernels.decode_form(gs_.to(DEV), mask_.to(DEV), bs, num_blocks, host_verdict=record, tag=tag)
        torch.cuda.synchronize()
        # the verdict the device published into pinned memory, under this call's tag
        assert int(record[0]) == (tag << 32 | int(bad.item()))
        return bt.cpu(), ctx.cpu(), int(bad.item())

    bt, ctx, bad = run(gs, mask)
    assert bad == 0 and ctx.tolist() == ctx_want
    for i, (tb, c) in enumerate(zip(tables, ctx_want)):
        assert bt[i, : metadata.blocks_for(c, bs)].tolist() == tb
    planted = []
    for r, k, value in ((0, t - 1, float("-inf")), (3, t - 1, float("nan")), (2, 100, -1.0), (1, 4500, torch.finfo(dtype).min)):
        m = mask.clone()
        m[r, 0, 0, k] = value
        planted.append(run(gs, m)[2])
    off_block = gs.clone()
    off_block[1, 4500] += 1
    planted.append(run(off_block, mask)[2])
    hidden = mask.clone()  # a row with no visible key: the mask kernel's uniform average, not ctx 0
    hidden[4, 0, 0, :] = torch.finfo(dtype).min
    planted.append(run(gs, hidden)[2])
    assert planted == [0, 1, 1, 1, 1, 1]
    # the capture form of the check zeroes every context length when it fails
    for m, ok in ((mask, True), (hidden, False)):
        _, ctx, bad = kernels.decode_form(gs.to(DEV), m.to(DEV), bs, num_blocks, clear_on_fail=True)
        torch.cuda.synchronize()
        assert int(bad.item()) == (0 if ok else 1)
        assert ctx.cpu().tolist() == (ctx_want if ok else [0] * len(ctx_want))


def test_reference_metadata_outside_the_decode_form_takes_the_mask_kernel():
    """A mask that hides a key inside the context, or slots that do not follow
    the block-table closed form, is not the decode form: the call reads
    gather_slots + mask as given (mask kernel) and matches the oracle's naive
    path on exactly that metadata."""
    bs, h_kv, n_rep, d = 16, 2, 4, 64
    num_cached = [40, 75, 3]
    tables = [list(range(i * 8, i * 8 + 8)) for i in range(3)]
    pool = PagedKVPool(1, 24, bs, h_kv, d, torch.float32, device=DEV)
    pool.k.normal_()
    pool.v.normal_()
    ours, mask = metadata.decode_context(pool, tables, num_cached)
    holed = mask.clone()
    holed[1, 0, 0, 10] = torch.finfo(torch.float32).min
    swapped = ours.gather_slots.clone()
    swapped[0, [3, 4]] = swapped[0, [4, 3]]
    for gs, m in ((ours.gather_slots, holed), (swapped, mask)):
        ref = _ReferenceContext(pool, ours.write_slots, gs)
        q = torch.randn(3, 1, h_kv * n_rep, d, device=DEV)
        k = torch.randn(3, 1, h_kv, d, device=DEV)
        v = torch.randn(3, 1, h_kv, d, device=DEV)
        got = paged_attention(q, k, v, ref, m, 0, d**-0.5, n_rep)
        torch.cuda.synchronize()
        assert pool._ref_form[1].verdict() is False  # published by the device, read without a wait
        again = paged_attention(q, k, v, ref, m, 0, d**-0.5, n_rep)  # the mask kernel alone now
        torch.cuda.synchronize()
        assert torch.equal(again, got)
        expect = O.paged_attention_naive(q.cpu(), pool.k[0].cpu(), pool.v[0].cpu(), gs.cpu(), m.cpu(), d**-0.5, n_rep)
        assert (got.cpu() - expect).abs().max().item() <= 1e-4


def _reference_prefill_frame(pool, tables, num_cached, q_lens, one_sequence_mask=False):
    """The reference engine's packed prefill frame, built by its own loops
    (infrared/engine/paged_engine.py:476-506, :194-206): per sequence the new
    tokens' write slots and its whole history's gather slots, and the mask of
    build_varlen_mask -- or, for one sequence, build_attention_mask
    (infrared/model/inputs.py:33-85; restated in the oracle)."""
    bs = pool.block_size
    write, gather, q_seq, q_pos, k_seq, k_pos = [], [], [], [], [], []
    for i, (bt, start, q) in enumerate(zip(tables, num_cached, q_lens)):
        for p in range(start, start + q):
            write.append(O.slot(bt, p, bs))
            q_seq.append(i)
            q_pos.append(p)
        for p in range(start + q):
            gather.append(O.slot(bt, p, bs))
            k_seq.append(i)
            k_pos.append(p)
    if one_sequence_mask:
        assert len(tables) == 1
        mask = O.attention_mask([0], num_cached[0], q_lens[0], num_cached[0] + q_lens[0], pool.dtype)
    else:
        mask = O.varlen_mask(torch.tensor(q_seq), torch.tensor(q_pos), torch.tensor(k_seq), torch.tensor(k_pos),
                             pool.dtype)
    return (torch.tensor(write, dtype=torch.int64, device=DEV), torch.tensor([gather], dtype=torch.int64, device=DEV),
            mask.to(DEV))


def _prefill_case(kind):
    g = torch.Generator().manual_seed(21)
    if kind == "prefix-hit":  # one sequence after a cached prefix
        num_cached, q_lens = [300], [77]
    elif kind == "mixed":  # two chunks (one after a prefix) and three decode rows
        num_cached, q_lens = [0, 300, 41, 1000, 7], [77, 130, 1, 1, 1]
    else:  # eight chunks after prefixes, enough work for the prefill plan
        num_cached = [int(x) for x in torch.randint(0, 2000, (8,), generator=g)]
        q_lens = [int(x) for x in torch.randint(64, 260, (8,), generator=g)]
    bs = 16
    need = [metadata.blocks_for(c + n, bs) for c, n in zip(num_cached, q_lens)]
    perm = torch.randperm(sum(need) + 40, generator=g).tolist()
    tables, off = [], 0
    for nb in need:
        tables.append(perm[off : off + nb])
        off += nb
    return tables, num_cached, q_lens, sum(need) + 40


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("kind", ["prefix-hit", "mixed", "chunks"])
def test_reference_prefill_metadata_runs_the_prefill_kernel(kind, dtype):
    """Unchanged reference callers pass a packed frame (batch 1) of gather_slots
    + the varlen / causal mask for prefix-hit prefills and mixed steps. Its
    form is recognised once per step (later layers reuse the derived metadata:
    cu_seqlens_q, q_start, block tables, and for a mixed step the split of its
    decode rows), and every layer equals the block-table context's output bit
    for bit -- the same kernels on the same metadata -- and the oracle (fp32:
    the fp32 prefill kernel, within 1e-4 of an fp64 restatement)."""
    tables, num_cached, q_lens, num_blocks = _prefill_case(kind)
    bs, h_kv, n_rep, d, layers = 16, 4, 7, 128, 3
    pool = PagedKVPool(layers, num_blocks, bs, h_kv, d, dtype, device=DEV)
    pool.k.normal_()
    pool.v.normal_()
    ours, _ = metadata.prefill_context(pool, tables, num_cached, q_lens)
    write, gather, mask = _reference_prefill_frame(pool, tables, num_cached, q_lens, kind == "prefix-hit")
    assert torch.equal(write, ours.write_slots)
    ref = _ReferenceContext(pool, write, gather)
    total = sum(q_lens)
    dgen = torch.Generator(device=DEV).manual_seed(2)
    forms = []
    for layer in range(layers):
        q = torch.randn(1, total, h_kv * n_rep, d, generator=dgen, device=DEV).to(dtype)
        k = torch.randn(1, total, h_kv, d, generator=dgen, device=DEV).to(dtype)
        v = torch.randn(1, total, h_kv, d, generator=dgen, device=DEV).to(dtype)
        got = paged_attention(q, k, v, ref, mask.to(dtype), layer, d**-0.5, n_rep)
        forms.append(pool._ref_varlen[1])
        want = paged_attention(q, k, v, ours, None, layer, d**-0.5, n_rep)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"layer {layer}"
        f32 = dtype == torch.float32
        expect = O.prefill_reference(q[0].cpu(), pool.k[layer].cpu(), pool.v[layer].cpu(),
                                     ours.block_tables.cpu(), ours.cu_seqlens_q.cpu(), num_cached, bs, d**-0.5,
                                     compute_dtype=torch.float64 if f32 else torch.float32)
        assert (got[0].to(expect.dtype).cpu() - expect).abs().max().item() <= (1e-4 if f32 else 2e-2)
    f = forms[0]
    assert f is not None and all(x is f for x in forms)
    assert f.max_q_len == max(q_lens)
    assert (f.row_split is not None) == (kind == "mixed")  # its decodes form one block of rows
    assert f.q_lens == tuple(q_lens) and f.prefixes == tuple(num_cached)
    assert torch.equal(f.cu_seqlens_q, ours.cu_seqlens_q) and torch.equal(f.q_start, ours.q_start)
    for i, (c, n) in enumerate(zip(num_cached, q_lens)):  # (entries past a history are never read)
        nb = metadata.blocks_for(c + n, bs)
        assert f.block_tables[i, :nb].tolist() == tables[i][:nb]


def test_reference_prefill_metadata_outside_the_form_takes_the_mask_kernel():
    """A frame that is not the reference's packed form -- a visible key hidden,
    a key of another sequence let through, two slots swapped, a mask value that
    is neither 0 nor a large negative, a key column no sequence owns -- is read
    as given (mask kernel) and matches the oracle's naive path on exactly that
    metadata."""
    tables, num_cached, q_lens, num_blocks = _prefill_case("mixed")
    bs, h_kv, n_rep, d = 16, 4, 7, 128
    pool = PagedKVPool(1, num_blocks, bs, h_kv, d, torch.bfloat16, device=DEV)
    pool.k.normal_()
    pool.v.normal_()
    write, gather, mask = _reference_prefill_frame(pool, tables, num_cached, q_lens)
    lo1 = num_cached[0] + q_lens[0]  # sequence 1's first key
    neg = torch.finfo(torch.bfloat16).min
    holed = mask.clone()
    holed[0, 0, 100, lo1 + 5] = neg  # row 100 is sequence 1's 24th query
    leaked = mask.clone()
    leaked[0, 0, 100, 3] = 0.0  # a key of sequence 0
    soft = mask.clone()
    soft[0, 0, 0, 70] = -1.0
    swapped = gather.clone()
    swapped[0, [lo1 + 3, lo1 + 4]] = swapped[0, [lo1 + 4, lo1 + 3]]
    extra_g = torch.cat([gather, gather[:, :1]], 1)
    extra_m = torch.cat([mask, torch.full_like(mask[..., :1], neg)], 3)
    total = sum(q_lens)
    for gs, m in ((gather, holed), (gather, leaked), (gather, soft), (swapped, mask), (extra_g, extra_m)):
        ref = _ReferenceContext(pool, write, gs)
        q = torch.randn(1, total, h_kv * n_rep, d, device=DEV).bfloat16()
        k = torch.randn(1, total, h_kv, d, device=DEV).bfloat16()
        v = torch.randn(1, total, h_kv, d, device=DEV).bfloat16()
        got = paged_attention(q, k, v, ref, m, 0, d**-0.5, n_rep)
        torch.cuda.synchronize()
        assert pool._ref_varlen[1] is None
        # the bar for a bf16 kernel: within 2e-2 of the same path in fp32
        expect = O.paged_attention_naive(q.float().cpu(), pool.k[0].float().cpu(), pool.v[0].float().cpu(),
                                         gs.cpu(), m.float().cpu(), d**-0.5, n_rep)
        assert (got.float().cpu() - expect).abs().max().item() <= 2e-2


@pytest.mark.parametrize("layout", ["flat", "misaligned", "strided"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_packed_form_check_reads_every_mask_layout(dtype, layout):
    """The packed-form check on masks of each dtype, stored contiguously from an
    aligned start (read as 16-byte pieces), from an unaligned start, or with a
    padded row stride (both read element by element). K and Q are odd, so rows
    start inside pieces and the array ends in a partial piece, and the longest
    history spans more than one pass of a row's loads. The derived metadata
    matches the frame; a NaN, a masked value above -6e4, a hidden key at the
    array's last element or inside the long history, and a leaked key at a
    row's first element each reject the frame, while -inf still masks; so do a
    slot off its block's closed form and a block outside the pool."""
    bs, num_cached, q_lens = 16, [0, 13, 26001], [5, 3, 5]
    need = [metadata.blocks_for(c + n, bs) for c, n in zip(num_cached, q_lens)]
    perm = torch.randperm(sum(need) + 7, generator=torch.Generator().manual_seed(5)).tolist()
    tables = [perm[sum(need[:i]) : sum(need[: i + 1])] for i in range(3)]
    q_seq, q_pos, k_seq, k_pos, gather = [], [], [], [], []
    for i, (bt, c, n) in enumerate(zip(tables, num_cached, q_lens)):
        q_seq += [i] * n
        q_pos += list(range(c, c + n))
        k_seq += [i] * (c + n)
        k_pos += list(range(c + n))
        gather += [O.slot(bt, p, bs) for p in range(c + n)]
    base = O.varlen_mask(torch.tensor(q_seq), torch.tensor(q_pos), torch.tensor(k_seq), torch.tensor(k_pos), dtype)
    Q, K = base.shape[2:]
    assert Q % 2 == 1 and K % 2 == 1
    gs = torch.tensor([gather], dtype=torch.int64, device=DEV)
    neg = torch.finfo(dtype).min
    long_key = 5 + 16 + 25000  # inside sequence 2's history, past a row's first pass of loads in every dtype

    def on_device(m):
        if layout == "flat":
            return m.to(DEV).contiguous()
        if layout == "misaligned":
            flat = torch.empty(Q * K + 1, dtype=dtype, device=DEV)
            flat[1:] = m.reshape(-1).to(DEV)
            return flat[1:].view(1, 1, Q, K)
        padded = torch.full((1, 1, Q, K + 3), neg, dtype=dtype, device=DEV)
        padded[..., :K] = m.to(DEV)
        return padded[..., :K]

    def planted(r, k, value):
        m = base.clone()
        m[0, 0, r, k] = value
        return m

    staging = torch.full((kernels.varlen_staging_size(Q),), -5, dtype=torch.int32, pin_memory=True)

    def forms(g, m):
        # the record copied back from device memory; written by the device into
        # pinned memory, tables in the call's capacity; the same with tables
        # wider than a capacity of one entry, written by the second launch
        return [kernels.varlen_form(g, m, bs, sum(need) + 7),
                kernels.varlen_form(g, m, bs, sum(need) + 7, staging=staging),
                kernels.varlen_form(g, m, bs, sum(need) + 7, staging=staging, tables_capacity=1)]

    for m, accepted in (
        (base, True),
        (planted(0, 100, float("-inf")), True),
        (planted(0, K - 1, float("nan")), False),
        (planted(Q - 1, 0, -1.0), False),
        (planted(Q - 1, K - 1, neg), False),
        (planted(8, long_key, neg), False),
        (planted(5, 0, 0.0), False),
    ):
        for f in forms(gs, on_device(m)):
            if not accepted:
                assert f is None
                continue
            assert f is not None
            assert f.q_lens == tuple(q_lens) and f.prefixes == tuple(num_cached) and f.max_q_len == max(q_lens)
            assert f.cu_seqlens_q.tolist() == [0, 5, 8, 13] and f.q_start.tolist() == num_cached
            assert f.block_tables.shape == (3, max(need))
            for i, nb in enumerate(need):
                assert f.block_tables[i, :nb].tolist() == tables[i]
                assert f.block_tables[i, nb:].eq(0).all()
    # slots the device check rejects: one off its block's closed form deep in
    # sequence 2, and a block head outside the pool
    off_form = gs.clone()
    off_form[0, long_key] += 1
    outside = gs.clone()
    outside[0, 5 + 16 + 25008 : 5 + 16 + 25024] += (sum(need) + 7) * bs  # one whole block, ids past the pool
    for bad_gs in (off_form, outside):
        assert forms(bad_gs, on_device(base)) == [None, None, None]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("case", [([0], [1]), ([0], [3]), ([2], [1]), ([0, 0], [1, 2]), ([1, 0, 3], [2, 1, 1])])
def test_packed_form_check_on_tiny_frames(dtype, case):
    """Frames of a few mask elements: shorter than one 16-byte piece (read
    element by element) or a whole piece followed by a partial one, where rows
    end in the partial piece."""
    num_cached, q_lens = case
    bs = 16
    tables = [[i] for i in range(len(q_lens))]
    q_seq, q_pos, k_seq, k_pos, gather = [], [], [], [], []
    for i, (c, n) in enumerate(zip(num_cached, q_lens)):
        q_seq += [i] * n
        q_pos += list(range(c, c + n))
        k_seq += [i] * (c + n)
        k_pos += list(range(c + n))
        gather += [O.slot(tables[i], p, bs) for p in range(c + n)]
    m = O.varlen_mask(torch.tensor(q_seq), torch.tensor(q_pos), torch.tensor(k_seq), torch.tensor(k_pos), dtype)
    f = kernels.varlen_form(torch.tensor([gather], dtype=torch.int64, device=DEV), m.to(DEV), bs, len(q_lens))
    assert f is not None
    assert f.q_lens == tuple(q_lens) and f.prefixes == tuple(num_cached)
    assert f.block_tables[:, 0].tolist() == [t[0] for t in tables]


def test_host_records_must_be_pinned():
    """The checks' host records are written by the device, so pageable memory
    is refused with an error (and the refusal is not left behind for the next
    call's launch check)."""
    gs = torch.tensor([[0, 1, 2]], dtype=torch.int64, device=DEV)
    m = torch.tensor([[[[0.0, 0.0, 0.0]]]], device=DEV)
    with pytest.raises(RuntimeError, match="not pinned host memory"):
        kernels.decode_form(gs, m, 16, 4, host_verdict=torch.zeros(1, dtype=torch.int64))
    bt, ctx, bad = kernels.decode_form(gs, m, 16, 4, host_verdict=torch.zeros(1, dtype=torch.int64, pin_memory=True))
    assert int(bad.item()) == 0 and ctx.tolist() == [3] and bt.tolist() == [[0]]
    frame = torch.zeros(1, 1, 1, 3, device=DEV)
    with pytest.raises(RuntimeError, match="not pinned host memory"):
        kernels.varlen_form(gs, frame, 16, 4, staging=torch.zeros(64, dtype=torch.int32))
    f = kernels.varlen_form(gs, frame, 16, 4, staging=torch.zeros(64, dtype=torch.int32, pin_memory=True))
    assert f is not None and f.q_lens == (1,) and f.prefixes == (2,)


def test_stream_handle_is_torchs_current_stream():
    """The launches' stream handle is torch's current stream: the default one,
    a side stream made current, and again the default one after it."""
    dev = torch.device(DEV, torch.cuda.current_device())
    assert stream_ptr(dev) == torch.cuda.current_stream(dev).cuda_stream
    side = torch.cuda.Stream(dev)
    with torch.cuda.stream(side):
        assert stream_ptr(dev) == side.cuda_stream != torch.cuda.default_stream(dev).cuda_stream
        assert stream_ptr(torch.device(DEV)) == side.cuda_stream
    assert stream_ptr(dev) == torch.cuda.current_stream(dev).cuda_stream


def test_a_host_record_that_never_arrives_raises(monkeypatch):
    """A record whose tag never comes (no call wrote it): the wait stops
    polling, synchronises the stream and raises rather than spinning on."""
    import numpy as np

    monkeypatch.setattr(kernels, "RECORD_POLLS", 50)
    host = np.zeros(16, dtype=np.int32)
    with pytest.raises(RuntimeError, match="wrote no record"):
        kernels.await_record(host, 7, 77, torch.device(DEV))


def test_packed_form_check_around_the_one_launch_row_limit():
    """Frames of 4,096 query rows (segmentation and slot check in one launch)
    and 4,097 rows (two launches): the derived metadata matches the frame in
    both, a leaked key rejects each, and so does a slot off its block's closed
    form; the host record of each call is that call's (one pinned record, the
    verdicts alternating)."""
    bs = 16
    staging = torch.zeros(kernels.varlen_staging_size(4097), dtype=torch.int32, pin_memory=True)
    for q_lens in ([2000, 1, 1595, 500], [2000, 1, 1596, 500]):
        num_cached = [0, 37, 5, 333]
        need = [metadata.blocks_for(c + n, bs) for c, n in zip(num_cached, q_lens)]
        perm = torch.randperm(sum(need) + 3, generator=torch.Generator().manual_seed(len(q_lens))).tolist()
        tables = [perm[sum(need[:i]) : sum(need[: i + 1])] for i in range(len(q_lens))]
        q_seq, q_pos, k_seq, k_pos, gather = [], [], [], [], []
        for i, (bt, c, n) in enumerate(zip(tables, num_cached, q_lens)):
            q_seq += [i] * n
            q_pos += list(range(c, c + n))
            k_seq += [i] * (c + n)
            k_pos += list(range(c + n))
            gather += [O.slot(bt, p, bs) for p in range(c + n)]
        mask = O.varlen_mask(torch.tensor(q_seq), torch.tensor(q_pos), torch.tensor(k_seq), torch.tensor(k_pos),
                             torch.bfloat16).to(DEV)
        assert mask.shape[2] == sum(q_lens) in (4096, 4097)
        gs = torch.tensor([gather], dtype=torch.int64, device=DEV)
        leaked = mask.clone()
        leaked[0, 0, 2500, 0] = 0.0  # a row of sequence 2 sees sequence 0's first key
        off_form = gs.clone()
        off_form[0, 2040] += 1
        for g, m, accepted in ((gs, mask, True), (gs, leaked, False), (off_form, mask, False), (gs, mask, True)):
            f = kernels.varlen_form(g, m, bs, sum(need) + 3, staging=staging)
            if not accepted:
                assert f is None
                continue
            assert f is not None and f.q_lens == tuple(q_lens) and f.prefixes == tuple(num_cached)
            assert f.max_q_len == max(q_lens)
            assert f.cu_seqlens_q.tolist() == [0, 2000, 2001, 2001 + q_lens[2], sum(q_lens)]
            assert f.q_start.tolist() == num_cached
            for i, nb in enumerate(need):
                assert f.block_tables[i, :nb].tolist() == tables[i]
                assert f.block_tables[i, nb:].eq(0).all()


def test_packed_form_check_on_a_key_axis_longer_than_one_pass_of_the_grid():
    """Two query rows over 300,000 keys (more keys than the verification's
    grid holds threads, so each thread checks several): the form is derived,
    its one table matches, and a slot off its closed form near the end of the
    axis -- in a later pass -- rejects the frame."""
    bs, prefix, q = 16, 299_998, 2
    k = prefix + q
    nb = -(-k // bs)
    table = torch.randperm(nb + 5, generator=torch.Generator().manual_seed(8))[:nb]
    pos = torch.arange(k)
    gs = (table[pos // bs] * bs + pos % bs).view(1, k).to(DEV)
    m = torch.full((1, 1, q, k), torch.finfo(torch.bfloat16).min, dtype=torch.bfloat16)
    m[0, 0, 0, : prefix + 1] = 0
    m[0, 0, 1, :] = 0
    m = m.to(DEV)
    staging = torch.zeros(kernels.varlen_staging_size(q), dtype=torch.int32, pin_memory=True)
    f = kernels.varlen_form(gs, m, bs, nb + 5, staging=staging)
    assert f is not None and f.q_lens == (q,) and f.prefixes == (prefix,)
    assert f.block_tables.shape == (1, nb) and torch.equal(f.block_tables[0].cpu(), table.to(torch.int32))
    bad = gs.clone()
    bad[0, k - 7] += 1
    assert kernels.varlen_form(bad, m, bs, nb + 5, staging=staging) is None
    assert kernels.varlen_form(gs, m, bs, nb + 5, staging=staging) is not None


def test_reference_metadata_refilled_in_place_is_checked_again():
    """A caller that reuses its gather_slots and mask tensors, refilling them in
    place for the next step, gets that step's form derived again (the cache of
    the step's check follows the tensors' in-place versions), not the last
    step's block tables and context lengths."""
    bs, h_kv, n_rep, d = 16, 4, 7, 128
    tables = [list(range(i * 32, i * 32 + 32)) for i in range(4)]
    pool = PagedKVPool(1, 128, bs, h_kv, d, torch.bfloat16, device=DEV)
    pool.k.normal_()
    pool.v.normal_()
    steps = [metadata.decode_context(pool, tables, nc) for nc in ([100, 300, 5, 400], [400, 12, 250, 99])]
    assert steps[0][0].gather_slots.shape == steps[1][0].gather_slots.shape
    gs, m = steps[0][0].gather_slots.clone(), steps[0][1].clone()
    for ours, mask in steps:
        gs.copy_(ours.gather_slots)
        m.copy_(mask)
        ref = _ReferenceContext(pool, ours.write_slots, gs)
        q = torch.randn(4, 1, h_kv * n_rep, d, device=DEV).bfloat16()
        k = torch.randn(4, 1, h_kv, d, device=DEV).bfloat16()
        v = torch.randn(4, 1, h_kv, d, device=DEV).bfloat16()
        got = paged_attention(q, k, v, ref, m, 0, d**-0.5, n_rep)
        torch.cuda.synchronize()
        form = pool._ref_form[1]
        assert form is not None and torch.equal(form.context_lens, ours.context_lens)
        expect = O.decode_reference(q[:, 0].cpu(), pool.k[0].cpu(), pool.v[0].cpu(), ours.block_tables.cpu(),
                                    ours.context_lens.cpu(), bs, d**-0.5)
        assert (got[:, 0].float().cpu() - expect).abs().max().item() <= 2e-2


@pytest.mark.parametrize("order", ["decodes-first", "decodes-last", "interleaved"])
def test_packed_step_runs_its_decode_rows_on_the_decode_kernels(order):
    """A packed step whose one-token rows form one block (packed first or last)
    is split: those rows run as a decode batch, the chunks as prefill, each
    writing its rows of the output in place; with the decodes interleaved
    among the chunks the step stays one prefill launch. Every layout matches
    the oracle."""
    g = torch.Generator().manual_seed(31)
    bs, h_kv, n_rep, d = 16, 4, 7, 128
    dec_cached = [int(x) for x in torch.randint(20, 900, (6,), generator=g)]
    chunks = [(0, 90), (300, 45)]
    if order == "decodes-first":
        seqs = [(c, 1) for c in dec_cached] + chunks
    elif order == "decodes-last":
        seqs = chunks + [(c, 1) for c in dec_cached]
    else:
        seqs = [chunks[0]] + [(c, 1) for c in dec_cached[:3]] + [chunks[1]] + [(c, 1) for c in dec_cached[3:]]
    num_cached, q_lens = [c for c, _ in seqs], [n for _, n in seqs]
    need = [metadata.blocks_for(c + n, bs) for c, n in seqs]
    perm = torch.randperm(sum(need) + 8, generator=g).tolist()
    tables, off = [], 0
    for nb in need:
        tables.append(perm[off : off + nb])
        off += nb
    pool = PagedKVPool(1, sum(need) + 8, bs, h_kv, d, torch.bfloat16, device=DEV, strict=True)
    pool.k.normal_()
    pool.v.normal_()
    paged, _ = metadata.prefill_context(pool, tables, num_cached, q_lens)
    assert (paged.row_split is None) == (order == "interleaved")
    total = sum(q_lens)
    q = torch.randn(1, total, h_kv * n_rep, d, device=DEV).bfloat16()
    k = torch.randn(1, total, h_kv, d, device=DEV).bfloat16()
    v = torch.randn(1, total, h_kv, d, device=DEV).bfloat16()
    out = paged_attention(q, k, v, paged, None, 0, d**-0.5, n_rep)
    torch.cuda.synchronize()
    bt = metadata.block_tables_tensor(tables, "cpu")
    ref = O.prefill_reference(q[0].cpu(), pool.k[0].cpu(), pool.v[0].cpu(), bt, paged.cu_seqlens_q.cpu(),
                              num_cached, bs, d**-0.5)
    assert (out[0].float().cpu() - ref).abs().max().item() <= 2e-2
