"""GPU parity of the chunked-prefill MFMA kernel (ir_paged_prefill, through the
C ABI) against the CPU oracle's per-sequence causal restatement
(oracle.naive.prefill_reference) on the same seeded inputs.

Bar: max-abs error <= 2e-2 for bf16/fp16 against the fp32 reference.
"""

from __future__ import annotations

import pytest
import torch

from infrared_amd import kernels
from infrared_amd._lib import ERR_BLOCK_RANGE, ERR_CONTEXT_RANGE
from infrared_amd.workloads import PrefillConfig, make_prefill_case
from oracle import naive as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
TOL = 2e-2


def _run(case, err=None, bt=None):
    cfg = case.config
    bt = case.block_tables[0] if bt is None else bt
    return kernels.paged_prefill(
        case.q, case.k_cache, case.v_cache, bt, case.cu_seqlens_q, case.q_start, max(case.q_lens),
        cfg.block_size, cfg.scale, err_flags=err,
    )


def _check(case):
    cfg = case.config
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = _run(case, err)
    torch.cuda.synchronize()
    assert err.item() == 0
    ref = O.prefill_reference(
        case.q.cpu(), case.k_cache.cpu(), case.v_cache.cpu(), case.block_tables[0].cpu(),
        case.cu_seqlens_q.cpu(), case.q_start.cpu(), cfg.block_size, cfg.scale,
    )
    diff = (out.float().cpu() - ref).abs().max().item()
    assert diff <= TOL, f"{cfg.name}: max-abs {diff}"
    return out


def test_prefill_qwen7b_full_size_parity():
    """8 x 512-token chunks after prefixes up to 8192 (pairs sharing prefix blocks)."""
    case = make_prefill_case("qwen7b-prefill", DEV)
    assert max(case.prefixes) > 2048
    _check(case)


def test_prefill_ragged_chunks_and_prefixes():
    """Chunks of 1..512 tokens after prefixes that end mid-block, one empty chunk."""
    case = make_prefill_case(
        "qwen7b-prefill", DEV, prefixes=[0, 37, 512, 1000, 3, 3, 0, 5], q_lens=[1, 31, 100, 512, 0, 9, 64, 33]
    )
    _check(case)


_SWEEP = [
    # (dtype, h_q, h_kv, d, bs)
    (torch.bfloat16, 28, 4, 128, 16),
    (torch.bfloat16, 8, 8, 64, 16),
    (torch.bfloat16, 16, 2, 128, 32),
    (torch.bfloat16, 24, 2, 64, 4),  # 12 heads per KV head: two head groups of 8
    (torch.float16, 28, 4, 128, 1),
    (torch.float16, 12, 3, 64, 8),
    # block sizes that are not powers of two take the general addressing path
    # (64-bit slot offsets, a division per key instead of shifts)
    (torch.bfloat16, 28, 4, 128, 12),
    (torch.float16, 8, 2, 64, 24),
]


@pytest.mark.parametrize("dtype,h_q,h_kv,d,bs", _SWEEP)
@pytest.mark.parametrize("layout", ["head_major", "slot_major"])
def test_prefill_shape_sweep(dtype, h_q, h_kv, d, bs, layout):
    """GQA groups 1..12 (one or two head groups per workgroup), both head dims,
    block sizes 1..32, both pool layouts, ragged chunks."""
    cfg = PrefillConfig(f"pf-{h_q}-{h_kv}-{d}-{bs}", 5, 0, h_q, h_kv, d, bs, dtype, 0, seed=h_q * d + bs)
    case = make_prefill_case(cfg, DEV, prefixes=[0, 17, 64, 200, 95], q_lens=[33, 64, 1, 130, 47], layout=layout)
    _check(case)


def test_prefill_workgroup_sizes_agree():
    """Small batches run 4-wavefront workgroups (128 query columns), large ones
    8 (256; the full-size test above): a 2-sequence batch on 4, and 160 query
    heads per KV head, which 4 wavefronts cannot hold, on 8 -- both match the
    oracle."""
    small = PrefillConfig("pf-small", 2, 0, 28, 4, 128, 16, torch.bfloat16, 0, seed=21)
    _check(make_prefill_case(small, DEV, prefixes=[0, 300], q_lens=[256, 77]))
    wide = PrefillConfig("pf-wide-group", 2, 0, 160, 1, 64, 16, torch.bfloat16, 0, seed=22)
    _check(make_prefill_case(wide, DEV, prefixes=[40, 0], q_lens=[5, 3]))


def test_prefill_block_id_cache_reload():
    """Block size 1 and a 2600-token context: the workgroup's staged block ids
    (1024 at a time) are refilled mid-walk."""
    cfg = PrefillConfig("pf-bs1-long", 2, 0, 8, 2, 64, 1, torch.bfloat16, 0, seed=3)
    _check(make_prefill_case(cfg, DEV, prefixes=[2500, 1100], q_lens=[100, 40]))


def test_prefill_packed_mixed_step_matches_decode_kernel():
    """A mixed step: 6 decode rows (one-token chunks) and 2 prefill chunks packed
    in one call. The decode rows also match the decode kernel on the same pool."""
    cfg = PrefillConfig("pf-mixed", 8, 0, 28, 4, 128, 16, torch.bfloat16, 0, seed=21)
    prefixes = [700, 1500, 99, 2047, 16, 3000, 0, 256]
    q_lens = [1, 1, 1, 1, 1, 1, 256, 200]
    case = make_prefill_case(cfg, DEV, prefixes=prefixes, q_lens=q_lens)
    out = _check(case)
    rows = [0, 1, 2, 3, 4, 5]
    q_dec = case.q[rows]
    ctx = torch.tensor([p + 1 for p in prefixes[:6]], dtype=torch.int32, device=DEV)
    dec = kernels.paged_decode(q_dec, case.k_cache, case.v_cache, case.block_tables[0][:6].contiguous(), ctx, 16,
                               cfg.scale)
    torch.cuda.synchronize()
    assert (dec.float() - out[rows].float()).abs().max().item() <= TOL


def test_prefill_deterministic():
    case = make_prefill_case("qwen7b-prefill", DEV, prefixes=[0, 40, 300, 1000, 5, 5, 0, 0],
                             q_lens=[512, 100, 64, 200, 1, 2, 3, 4])
    a = _run(case)
    b = _run(case)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_prefill_flags_bad_block_ids_and_overlong_context():
    case = make_prefill_case("qwen7b-prefill", DEV, prefixes=[32, 0, 0, 0, 0, 0, 0, 0], q_lens=[16] * 8)
    bt = case.block_tables[0].clone()
    bt[0, 1] = case.pool_blocks + 7  # key 16..31 of sequence 0: outside the pool
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    _run(case, err, bt)
    torch.cuda.synchronize()
    assert err.item() & ERR_BLOCK_RANGE
    # a chunk reaching past what its table can hold
    err.zero_()
    qs = case.q_start.clone()
    qs[1] = bt.shape[1] * 16
    kernels.paged_prefill(case.q, case.k_cache, case.v_cache, case.block_tables[0], case.cu_seqlens_q, qs, 16, 16,
                          case.config.scale, err_flags=err)
    torch.cuda.synchronize()
    assert err.item() & ERR_CONTEXT_RANGE


F32_TOL = 1e-4  # the fp32 bar, against an fp64 restatement

_F32_SWEEP = [
    # (h_q, h_kv, d, bs): the 0.5B model's shape; one query head per KV head;
    # GQA 7 at head_dim 128 on a 12-token block (general addressing); 64 query
    # heads per KV head (one token per workgroup)
    (14, 2, 64, 16),
    (8, 8, 128, 16),
    (28, 4, 128, 12),
    (64, 1, 64, 16),
]


def _check_f32(case, plan=None):
    cfg = case.config
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = kernels.paged_prefill(case.q, case.k_cache, case.v_cache, case.block_tables[0], case.cu_seqlens_q,
                                case.q_start, max(case.q_lens), cfg.block_size, cfg.scale, err_flags=err, plan=plan)
    torch.cuda.synchronize()
    assert err.item() == 0
    ref = O.prefill_reference(case.q.cpu(), case.k_cache.cpu(), case.v_cache.cpu(), case.block_tables[0].cpu(),
                              case.cu_seqlens_q.cpu(), case.q_start.cpu(), cfg.block_size, cfg.scale,
                              compute_dtype=torch.float64)
    diff = (out.double().cpu() - ref).abs().max().item()
    assert diff <= F32_TOL, f"{cfg.name}: max-abs {diff}"
    return out


@pytest.mark.parametrize("h_q,h_kv,d,bs", _F32_SWEEP)
@pytest.mark.parametrize("layout", ["head_major", "slot_major"])
def test_prefill_fp32_matches_the_oracle(h_q, h_kv, d, bs, layout):
    """fp32 chunks -- the reference's fp32 path -- on their own kernel: ragged
    chunks after prefixes that end mid-block, both pool layouts, within 1e-4
    of an fp64 restatement."""
    cfg = PrefillConfig(f"pf32-{h_q}-{h_kv}-{d}-{bs}", 5, 0, h_q, h_kv, d, bs, torch.float32, 0, seed=h_q + d + bs)
    case = make_prefill_case(cfg, DEV, prefixes=[0, 17, 64, 200, 95], q_lens=[33, 64, 1, 130, 47], layout=layout)
    _check_f32(case)


def _cut_entries(plan, n):
    """nparts of the plan's first n entries (heaviest first)."""
    items = plan.buf[: 8 * n].view(torch.int32).view(n, 2).cpu()
    return (items[:, 1] & 0xFF).tolist()


def test_prefill_fp32_reloads_block_ids_and_runs_its_plan():
    """fp32, block size 1 and a 2,600-token context: the staged block ids are
    refilled mid-walk. A plan built for fp32 (IR_PLAN_F32) cuts the long items
    into key-range pieces: within 1e-4 of the restatement, within fp32 merge
    rounding of the unplanned call, and the same bit for bit on a second call
    (its arrival counters reset); a 16-bit plan is refused."""
    cfg = PrefillConfig("pf32-bs1-long", 2, 0, 8, 2, 64, 1, torch.float32, 0, seed=3)
    case = make_prefill_case(cfg, DEV, prefixes=[2500, 1100], q_lens=[100, 40])
    out = _check_f32(case)
    plan = kernels.prefill_plan(case.cu_seqlens_q, case.q_start, case.block_tables[0], case.q.shape[0], 100,
                                cfg.block_size, cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim, dtype=torch.float32)
    assert plan.f32 and max(_cut_entries(plan, 8)) > 1  # the heaviest items are cut
    planned = _check_f32(case, plan)
    assert (planned - out).abs().max().item() <= 1e-5
    assert torch.equal(_check_f32(case, plan), planned)
    plan16 = kernels.prefill_plan(case.cu_seqlens_q, case.q_start, case.block_tables[0], case.q.shape[0], 100,
                                  cfg.block_size, cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim)
    with pytest.raises(RuntimeError, match="16-bit"):
        _check_f32(case, plan16)


def test_prefill_fp32_planned_long_prefixes():
    """fp32 chunks after long prefixes that pairs share, and an empty chunk, on
    a plan: cut items merged within 1e-4 of the restatement, and a plan
    placing share groups gives the same outputs bit for bit (the placement
    changes the schedule only)."""
    cfg = PrefillConfig("pf32-plan", 5, 0, 28, 4, 128, 16, torch.float32, 0, seed=21)
    case = make_prefill_case(cfg, DEV, prefixes=[3000, 3500, 200, 5000, 64], q_lens=[64, 17, 96, 40, 0])
    outs = []
    for share_groups in (False, True):
        plan = kernels.prefill_plan(case.cu_seqlens_q, case.q_start, case.block_tables[0], case.q.shape[0], 96,
                                    cfg.block_size, cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim,
                                    share_groups=share_groups, dtype=torch.float32)
        assert max(_cut_entries(plan, 8)) > 1
        outs.append(_check_f32(case, plan))
    assert torch.equal(outs[0], outs[1])


def test_prefill_fp32_flags_bad_block_ids_and_refuses_wide_groups():
    """fp32: a block id outside the pool is flagged and its keys read as zeros
    (within 1e-4 of the restatement with that block zeroed); more than 64 query
    heads per KV head are refused."""
    cfg = PrefillConfig("pf32-bad", 3, 0, 14, 2, 64, 16, torch.float32, 0, seed=12)
    case = make_prefill_case(cfg, DEV, prefixes=[40, 300, 0], q_lens=[20, 50, 70])
    bt = case.block_tables[0].clone()
    bt[1, 2] = case.pool_blocks + 9
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = kernels.paged_prefill(case.q, case.k_cache, case.v_cache, bt, case.cu_seqlens_q, case.q_start, 70,
                                cfg.block_size, cfg.scale, err_flags=err)
    torch.cuda.synchronize()
    assert err.item() == ERR_BLOCK_RANGE
    kz, vz = case.k_cache.clone().cpu(), case.v_cache.clone().cpu()
    zero_bt = bt.cpu().clone()
    zero_bt[1, 2] = case.pool_blocks  # an extra all-zero block appended below
    kz = torch.cat([kz, torch.zeros(cfg.block_size, *kz.shape[1:])])
    vz = torch.cat([vz, torch.zeros(cfg.block_size, *vz.shape[1:])])
    ref = O.prefill_reference(case.q.cpu(), kz, vz, zero_bt, case.cu_seqlens_q.cpu(), case.q_start.cpu(),
                              cfg.block_size, cfg.scale, compute_dtype=torch.float64)
    assert (out.double().cpu() - ref).abs().max().item() <= F32_TOL
    wide = PrefillConfig("pf32-wide", 1, 0, 128, 1, 64, 16, torch.float32, 0, seed=13)
    case = make_prefill_case(wide, DEV, prefixes=[5], q_lens=[3])
    with pytest.raises(RuntimeError, match="fp32 with more than 64"):
        kernels.paged_prefill(case.q, case.k_cache, case.v_cache, case.block_tables[0], case.cu_seqlens_q,
                              case.q_start, 3, wide.block_size, wide.scale)


def _host_weights(case, tq, n_qblocks):
    """Key tiles (64 keys) each (sequence, query block) item walks, -1 for items
    without query rows: the bounds the prefill kernel applies, from the host
    copy of the metadata."""
    cap = case.block_tables[0].shape[1] * case.config.block_size
    cu = case.cu_seqlens_q.cpu().tolist()
    qs = case.q_start.cpu().tolist()
    w = []
    for b in range(len(qs)):
        q_len = cu[b + 1] - cu[b]
        for tb in range(n_qblocks):
            if tb * tq >= q_len:
                w.append(-1)
                continue
            p0 = max(0, min(qs[b], cap))
            kmax = min(cap, p0 + min(q_len, (tb + 1) * tq))
            w.append((kmax + 63) // 64)
    return w


def _plan_geometry(b, max_q, hq, hkv):
    """Items, entries and piece capacity of a plan: 4-wavefront workgroups of
    128 // n_rep query tokens, two resident per CU, the capacity one piece per
    KV head of every workgroup slot; one entry per workgroup, (items +
    capacity) x KV heads, 1.5x that rounded to the XCD count when the plan
    places work on XCDs."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    tq = 128 // (hq // hkv)
    n_qblocks = -(-max_q // tq)
    slots = 2 * cus
    cap = -(-slots // hkv)
    wgs = (b * n_qblocks + cap) * hkv
    x = kernels.prefill_plan_xcds()
    entries = x * -(-(wgs * 3 // 2) // x) if x > 1 else wgs
    return tq, n_qblocks, slots, cap, entries, x


def _plan_entries(plan, entries):
    return plan.buf[: entries * 8].view(torch.int32).view(entries, 2).cpu().tolist()


def _plan_order(rows, h_kv, x, w):
    """How the plan placed its workgroups: "slots" -- rows of x entries, each
    row holding one piece per slot of h_kv consecutive entries (its KV heads
    in order), every slot's pieces in non-increasing weight and then empty --
    or "global" -- the pieces in non-increasing weight, a piece's KV heads on
    consecutive entries, then empty entries. None if neither."""
    def weight(e, piece):
        return -(-w[e // h_kv] // (piece & 0xFF))

    def one_piece(grp):
        return len({(e // h_kv, p) for e, p in grp}) == 1 and [e % h_kv for e, _ in grp] == list(range(h_kv))

    used = sum(1 for e, _ in rows if e >= 0)
    if all(e >= 0 for e, _ in rows[:used]) and all(e < 0 for e, _ in rows[used:]) and used % h_kv == 0:
        pieces = [rows[k * h_kv:(k + 1) * h_kv] for k in range(used // h_kv)]
        if all(one_piece(grp) for grp in pieces):
            ws = [weight(*grp[0]) for grp in pieces]
            if ws == sorted(ws, reverse=True):
                return "global"
    if h_kv < x and x % h_kv == 0 and len(rows) % x == 0:
        for sl in range(x // h_kv):
            ws = []
            for r in range(len(rows) // x):
                grp = rows[r * x + sl * h_kv: r * x + (sl + 1) * h_kv]
                if all(e < 0 for e, _ in grp):
                    ws.append(None)
                    continue
                if not one_piece(grp):
                    return None
                ws.append(weight(*grp[0]))
            n = sum(1 for v in ws if v is not None)
            if any(v is None for v in ws[:n]) or ws[:n] != sorted(ws[:n], reverse=True):
                return None
        return "slots"
    return None


@pytest.mark.parametrize("prefixes,q_lens", [
    (None, None),  # the full 8 x 512-token workload, sequence pairs sharing their prefix blocks
    ([0, 37, 512, 1000, 3, 3, 0, 5], [1, 31, 100, 512, 0, 9, 64, 33]),  # ragged, one empty chunk
    ([0, 300], [256, 77]),  # few workgroups, nothing cut
    ([9000, 0, 0, 0], [512, 40, 40, 40]),  # one very long item among short ones
])
@pytest.mark.parametrize("share_groups", [False, True])
def test_prefill_plan_covers_every_item_heaviest_first(prefixes, q_lens, share_groups):
    """The device-built plan lists every (item with work, KV head) exactly once
    per piece -- whole, or as nparts pieces numbered 0..nparts-1 sharing one
    block of partial rows (blocks disjoint, inside the capacity) -- and empty
    entries elsewhere. Items heavier than the mean load of a workgroup slot x
    1.5 (raised until the pieces fit the plan's capacity) are cut, and no piece
    is heavier than that threshold. Order: one global heaviest-first order,
    or, with share groups placed, rows of X entries holding one piece per slot
    of 4 consecutive XCDs, every slot heaviest first (the weights here are
    below the 256 weight ranges, so the order is exact). With share groups on
    the full workload the plan keeps each (sequence pair, KV head) -- the pairs
    share their prefix blocks -- on one XCD."""
    cfg = PrefillConfig("pf-plan", 8 if prefixes is None else len(prefixes), 512, 28, 4, 128, 16,
                        torch.bfloat16, 8192, seed=4)
    case = make_prefill_case(cfg, DEV, prefixes=prefixes, q_lens=q_lens)
    b, max_q = len(case.q_lens), max(case.q_lens)
    tq, n_qblocks, slots, cap, entries, x = _plan_geometry(b, max_q, 28, 4)
    plan = kernels.prefill_plan(case.cu_seqlens_q, case.q_start, case.block_tables[0], case.q.shape[0], max_q,
                                16, 28, 4, 128, share_groups=share_groups)
    assert plan.buf.numel() >= entries * 8
    rows = _plan_entries(plan, entries)
    w = _host_weights(case, tq, n_qblocks)
    total = sum(x_ for x_ in w if x_ > 0)

    def pieces(x_, t):
        return min(16, -(-x_ // t)) if x_ > t else (1 if x_ >= 0 else 0)

    # the cut threshold: 1.5x the mean load of a workgroup slot (at least 8
    # tiles), raised to the smallest value whose cut pieces fit the capacity
    thresh = max(8, -(-total * 4 * 3 // (2 * slots)))
    while sum(pieces(x_, thresh) for x_ in w if x_ > thresh) > cap:
        thresh += 1
    seen, blocks, piece_w = {}, set(), []
    for e, piece in rows:
        if e < 0:
            assert piece == 0
            continue
        item, head = divmod(e, 4)
        np_, part, pb = piece & 0xFF, (piece >> 8) & 0xFF, piece >> 16
        seen.setdefault((item, head), []).append((np_, part, pb))
        piece_w.append(-(-w[item] // np_))
    assert sorted(seen) == [(i, h) for i in range(len(w)) if w[i] >= 0 for h in range(4)]
    for (item, head), parts in seen.items():
        np_ = parts[0][0]
        assert sorted(p for _, p, _ in parts) == list(range(np_)) and len({(n, b_) for n, _, b_ in parts}) == 1
        assert parts[0][::2] == seen[(item, 0)][0][::2], "every KV head of an item is cut alike"
        if np_ > 1 and head == 0:
            pb = parts[0][2]
            assert pb + np_ <= cap and not blocks & set(range(pb, pb + np_))
            blocks |= set(range(pb, pb + np_))
        assert (np_ > 1) == (w[item] > thresh)
    assert max(piece_w) <= thresh
    order = _plan_order(rows, 4, x, w)
    assert order == "global" if not share_groups else order is not None
    if prefixes is not None and prefixes[0] == 9000:
        assert blocks, "the heaviest items of this workload must be cut"
    if share_groups and prefixes is None and x > 4 and x % 4 == 0:
        assert order == "slots"
        xcds = {}
        for k, (e, _) in enumerate(rows):
            if e >= 0:
                item, head = divmod(e, 4)
                xcds.setdefault((item // n_qblocks // 2, head), set()).add(k % x)
        assert all(len(v) == 1 for v in xcds.values()), xcds


def test_prefill_plan_results_match_the_unplanned_call():
    """The same calls with and without a plan: equal outputs (bit for bit where
    no item is cut; within fp32 rounding of the log-sum-exp merge where one is)
    and the same error flags -- the full workload, ragged chunks, a packed
    mixed step, bad block ids -- and each within the bar of the oracle; a plan
    placing share groups gives the default plan's outputs bit for bit."""
    cases = [
        make_prefill_case("qwen7b-prefill", DEV),
        make_prefill_case("qwen7b-prefill", DEV, prefixes=[0, 37, 512, 1000, 3, 3, 0, 5],
                          q_lens=[1, 31, 100, 512, 0, 9, 64, 33]),
        make_prefill_case(PrefillConfig("pf-mixed-o", 8, 0, 28, 4, 128, 16, torch.bfloat16, 0, seed=21), DEV,
                          prefixes=[700, 1500, 99, 2047, 16, 3000, 0, 256], q_lens=[1, 1, 1, 1, 1, 1, 256, 200]),
        make_prefill_case(PrefillConfig("pf-long", 4, 0, 28, 4, 128, 16, torch.bfloat16, 0, seed=23), DEV,
                          prefixes=[9000, 0, 17, 0], q_lens=[512, 40, 40, 300]),
    ]
    for i, case in enumerate(cases):
        cfg = case.config
        bt = case.block_tables[0].clone()
        if i == 1:
            bt[3, 5] = case.pool_blocks + 3  # a bad block id inside sequence 3's keys
        b, max_q = len(case.q_lens), max(case.q_lens)
        plan = kernels.prefill_plan(case.cu_seqlens_q, case.q_start, bt, case.q.shape[0], max_q,
                                    cfg.block_size, cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim)
        plan_g = kernels.prefill_plan(case.cu_seqlens_q, case.q_start, bt, case.q.shape[0], max_q,
                                      cfg.block_size, cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim,
                                      buf=torch.empty_like(plan.buf), share_groups=True)
        outs, errs = [], []
        for pl in (None, plan, plan_g):
            err = torch.zeros(1, dtype=torch.int32, device=DEV)
            outs.append(kernels.paged_prefill(case.q, case.k_cache, case.v_cache, bt, case.cu_seqlens_q,
                                              case.q_start, max_q, cfg.block_size, cfg.scale, err_flags=err,
                                              plan=pl))
            errs.append(err)
        torch.cuda.synchronize()
        assert errs[0].item() == errs[1].item() == errs[2].item() == (ERR_BLOCK_RANGE if i == 1 else 0)
        # the placement changes the schedule only: both plans give identical outputs
        assert torch.equal(outs[1], outs[2]), cfg.name
        cut = any((piece & 0xFF) > 1 for item, piece in _plan_entries(
            plan, _plan_geometry(b, max_q, cfg.num_q_heads, cfg.num_kv_heads)[4]) if item >= 0)
        assert cut or i != 3, f"{cfg.name}: its heaviest items must be cut"
        if cut:
            assert (outs[0].float() - outs[1].float()).abs().max().item() <= TOL, cfg.name
        else:
            assert torch.equal(outs[0], outs[1]), cfg.name
        if i != 1:
            ref = O.prefill_reference(case.q.cpu(), case.k_cache.cpu(), case.v_cache.cpu(), bt.cpu(),
                                      case.cu_seqlens_q.cpu(), case.q_start.cpu(), cfg.block_size, cfg.scale)
            assert (outs[1].float().cpu() - ref).abs().max().item() <= TOL, cfg.name


def test_prefill_plan_size_is_checked():
    case = make_prefill_case("qwen7b-prefill", DEV)
    cfg = case.config
    small = kernels.PrefillPlan(torch.empty(1024, dtype=torch.uint8, device=DEV), cfg.num_seqs, cfg.chunk,
                                cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim)
    with pytest.raises(RuntimeError, match="plan of"):
        kernels.paged_prefill(case.q, case.k_cache, case.v_cache, case.block_tables[0], case.cu_seqlens_q,
                              case.q_start, cfg.chunk, cfg.block_size, cfg.scale, plan=small)


_SCHED_CHILD = r"""
import sys, torch
sys.path.insert(0, {root!r})
sys.path.insert(0, {tests!r})
from test_gpu_prefill import _SCHED_CASES, _run
from infrared_amd.workloads import make_prefill_case
name, prefixes, q_lens = _SCHED_CASES[{key!r}]
out = _run(make_prefill_case(name, "cuda", prefixes=prefixes, q_lens=q_lens))
torch.cuda.synchronize()
torch.save(out.cpu(), {path!r})
print("SCHED OK")
"""

_SCHED_CASES = {
    "c4": ("qwen7b-prefill", None, None),
    "ragged": ("qwen7b-prefill", [0, 37, 512, 1000, 3, 3, 0, 5], [1, 31, 100, 512, 0, 9, 64, 33]),
    # fp16, head_dim 64, a 12-token block (general addressing path)
    "f16-bs12": (PrefillConfig("pf-s-f16", 8, 0, 32, 8, 64, 12, torch.float16, 0, seed=31),
                 [0, 100, 7, 300, 12, 0, 50, 1], [300, 256, 290, 200, 310, 280, 260, 299]),
    # grids no larger than the CUs (240 and 48 workgroups): 8 wavefronts of one column tile by default
    "small": (PrefillConfig("pf-small", 4, 256, 28, 4, 128, 16, torch.bfloat16, 0, seed=7),
              [0, 100, 700, 33], [256, 256, 256, 256]),
    "small-f16": (PrefillConfig("pf-small-f16", 3, 64, 32, 8, 64, 12, torch.float16, 0, seed=9),
                  [0, 50, 300], [64, 1, 40]),
}


@pytest.mark.parametrize("key", list(_SCHED_CASES))
def test_prefill_schedules_agree_bit_for_bit(key, tmp_path):
    """Every workgroup shape and schedule does each column's arithmetic in the
    same order: 4-wavefront workgroups on the 2-deep ring, on the 3-deep ring
    (next tile's scores beside this tile's exponentials), 8-wavefront
    workgroups, and -- on grids no larger than the CUs, where it is the
    default -- 8 wavefronts of one column tile give identical outputs, within
    the bar of the oracle. The knobs are read once per process, so each shape
    runs in a child process."""
    import os
    import subprocess
    import sys

    name, prefixes, q_lens = _SCHED_CASES[key]
    tests = os.path.dirname(os.path.abspath(__file__))
    outs = []
    envs = ({"IR_PREFILL_RING2": "1"}, {"IR_PREFILL_RING2": "0", "IR_PREFILL_SPLIT": "0"}, {"IR_PREFILL_WAVES": "8"},
            {"IR_PREFILL_SPLIT": "0"})
    for i, env in enumerate(envs):
        path = str(tmp_path / f"s{i}.pt")
        res = subprocess.run(
            [sys.executable, "-c", _SCHED_CHILD.format(root=os.path.dirname(tests), tests=tests, key=key, path=path)],
            env={**os.environ, **env}, capture_output=True, text=True, timeout=110,
        )
        assert res.returncode == 0 and "SCHED OK" in res.stdout, str(env) + res.stdout + res.stderr[-2000:]
        outs.append(torch.load(path, weights_only=True))
    assert all(torch.equal(outs[0], o) for o in outs[1:])
    case = make_prefill_case(name, DEV, prefixes=prefixes, q_lens=q_lens)
    cfg = case.config
    ref = O.prefill_reference(
        case.q.cpu(), case.k_cache.cpu(), case.v_cache.cpu(), case.block_tables[0].cpu(),
        case.cu_seqlens_q.cpu(), case.q_start.cpu(), cfg.block_size, cfg.scale,
    )
    assert (outs[0].float() - ref).abs().max().item() <= TOL


def test_prefill_flags_understated_max_q_len():
    """A chunk longer than the host's max_q_len bound has rows no workgroup
    covers: the call flags IR_ERR_CONTEXT_RANGE instead of leaving them silently
    unwritten; with the true bound the same call is clean."""
    case = make_prefill_case("qwen7b-prefill", DEV, prefixes=[0, 64, 0, 0, 0, 0, 0, 0],
                             q_lens=[300, 40, 8, 8, 8, 8, 8, 8])
    cfg = case.config
    for max_q, flagged in ((100, True), (300, False)):
        err = torch.zeros(1, dtype=torch.int32, device=DEV)
        kernels.paged_prefill(case.q, case.k_cache, case.v_cache, case.block_tables[0], case.cu_seqlens_q,
                              case.q_start, max_q, cfg.block_size, cfg.scale, err_flags=err)
        torch.cuda.synchronize()
        assert bool(err.item() & ERR_CONTEXT_RANGE) == flagged, (max_q, err.item())


@pytest.mark.parametrize("share_groups", [False, True])
def test_prefill_plan_and_kernel_replay_in_a_hip_graph(share_groups):
    """A step's plan build and prefill captured in one hipGraph: each of three
    replays -- with eager work clearing the output and scribbling over the plan
    buffer in between -- equals the eager planned call bit for bit. Default
    placement: one 9,000-token prefix among short ones, whose heaviest items are
    cut and merged through the plan's counters; share groups: the 8 x 512-token
    workload, whose sequence pairs share prefix blocks."""
    if share_groups:
        case = make_prefill_case("qwen7b-prefill", DEV)
    else:
        case = make_prefill_case(PrefillConfig("pf-long-g", 4, 0, 28, 4, 128, 16, torch.bfloat16, 0, seed=23), DEV,
                                 prefixes=[9000, 0, 17, 0], q_lens=[512, 40, 40, 300])
    cfg = case.config
    b, max_q = len(case.q_lens), max(case.q_lens)
    buf = torch.empty(kernels.prefill_plan_bytes(b, max_q, cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim),
                      dtype=torch.uint8, device=DEV)
    out = torch.empty_like(case.q)

    def call():
        plan = kernels.prefill_plan(case.cu_seqlens_q, case.q_start, case.block_tables[0], case.q.shape[0], max_q,
                                    cfg.block_size, cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim, buf=buf,
                                    share_groups=share_groups)
        kernels.paged_prefill(case.q, case.k_cache, case.v_cache, case.block_tables[0], case.cu_seqlens_q,
                              case.q_start, max_q, cfg.block_size, cfg.scale, out=out, plan=plan)

    call()
    torch.cuda.synchronize()
    eager = out.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for _ in range(3):
        out.zero_()
        buf.fill_(7)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
