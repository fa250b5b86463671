"""The chunked-prefill kernel with the step's K/V write folded into its launch
(ir_paged_prefill with k_new / v_new / write_slots, through the C ABI) against
the two launches it replaces: ir_kv_scatter of the same rows, then the
unfused ir_paged_prefill. The attention output must be identical bit for bit
(the call reads its own new keys from the rows it is given, which hold the
values the scatter would have stored) and so must the pool afterwards, for
every workgroup shape (the small-grid 8 x 1 shape, 4-wavefront workgroups,
planned calls with cut items, the general addressing path), with rows of
other sequences before the call's own, skipped (negative) slots included.
A new token whose write slot is not its block-table slot is flagged."""

from __future__ import annotations

import pytest
import torch

from infrared_amd import kernels
from infrared_amd._lib import ERR_WRITE_SLOT
from infrared_amd.workloads import PrefillConfig, make_prefill_case
from oracle import naive as O

pytestmark = pytest.mark.gpu
DEV = "cuda"

CASES = {
    # 240 workgroups: one per CU, 8 wavefronts of one column tile
    "small": (PrefillConfig("fw-small", 4, 256, 28, 4, 128, 16, torch.bfloat16, 0, seed=3),
              [0, 100, 700, 33], [256, 256, 256, 256], False),
    # 928 workgroups, no plan: 4-wavefront workgroups in index order
    "unplanned": (PrefillConfig("fw-unplanned", 8, 512, 28, 4, 128, 16, torch.bfloat16, 0, seed=4),
                  [2110, 3183, 2335, 290, 4017, 335, 5780, 673], [512] * 8, False),
    # the same with the work plan (long items cut, pieces merged)
    "planned": (PrefillConfig("fw-planned", 8, 512, 28, 4, 128, 16, torch.bfloat16, 0, seed=4),
                [2110, 3183, 2335, 290, 4017, 335, 5780, 673], [512] * 8, True),
    # fp16, head_dim 64, a 12-token block (general addressing path)
    "f16-bs12": (PrefillConfig("fw-f16", 5, 0, 32, 8, 64, 12, torch.float16, 0, seed=5),
                 [0, 100, 7, 300, 12], [300, 1, 290, 64, 31], False),
}


def _frame(key):
    cfg, prefixes, q_lens, planned = CASES[key]
    case = make_prefill_case(cfg, DEV, prefixes=prefixes, q_lens=q_lens)
    bs, h_kv, d = cfg.block_size, cfg.num_kv_heads, cfg.head_dim
    bt = case.block_tables[0]
    rows = bt.cpu().tolist()
    # the call's own rows: each new token's slot from its block table
    own = [O.slot(rows[i], p, bs) for i, (p0, n) in enumerate(zip(prefixes, q_lens)) for p in range(p0, p0 + n)]
    # rows of other sequences first (decode-like rows): slots in blocks no table uses, two skipped
    num_blocks = case.k_cache.shape[0] // bs
    used = {b for i, (p0, n) in enumerate(zip(prefixes, q_lens)) for b in rows[i][: -(-(p0 + n) // bs)]}
    free = [b for b in range(num_blocks) if b not in used]
    extra = [free[j % len(free)] * bs + (j // len(free)) % bs for j in range(37)]
    extra[5] = extra[20] = -1
    spare = free[-1] * bs + bs - 1  # a slot no row writes
    assert 37 // len(free) < bs - 1
    slots = torch.tensor(extra + own, dtype=torch.int64, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(11)
    n = slots.shape[0]
    k_new = torch.randn(n, h_kv, d, generator=g, device=DEV).to(cfg.dtype)
    v_new = torch.randn(n, h_kv, d, generator=g, device=DEV).to(cfg.dtype)
    plan = None
    if planned:
        plan = kernels.prefill_plan(case.cu_seqlens_q, case.q_start, bt, case.q.shape[0], max(q_lens), bs,
                                    cfg.num_q_heads, h_kv, d)
    return case, bt, slots, k_new, v_new, len(extra), plan, spare


@pytest.mark.parametrize("key", list(CASES))
def test_fused_write_equals_scatter_then_prefill(key):
    case, bt, slots, k_new, v_new, row0, plan, _ = _frame(key)
    cfg = case.config
    max_q = max(CASES[key][2])
    kc0, vc0 = case.k_cache.clone(), case.v_cache.clone()
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    kernels.kv_scatter(case.k_cache, case.v_cache, k_new, v_new, slots, err)
    want = kernels.paged_prefill(case.q, case.k_cache, case.v_cache, bt, case.cu_seqlens_q, case.q_start, max_q,
                                 cfg.block_size, cfg.scale, err_flags=err, plan=plan)
    torch.cuda.synchronize()
    assert err.item() == 0
    kc, vc = case.k_cache.clone(), case.v_cache.clone()
    case.k_cache.copy_(kc0)
    case.v_cache.copy_(vc0)
    for rep in range(2):  # the second call on the same plan: counters back at zero
        got = kernels.paged_prefill(case.q, case.k_cache, case.v_cache, bt, case.cu_seqlens_q, case.q_start, max_q,
                                    cfg.block_size, cfg.scale, err_flags=err, plan=plan,
                                    new_kv=(k_new, v_new, slots), src_row0=row0)
        torch.cuda.synchronize()
        assert err.item() == 0
        assert torch.equal(got, want), f"{key}: call {rep} differs from scatter + prefill"
        assert torch.equal(case.k_cache, kc) and torch.equal(case.v_cache, vc), f"{key}: pool differs"


def test_fused_write_flags_a_token_written_elsewhere():
    """A new token whose write slot is not its block-table slot: the row goes
    where the slot says, the call attends the row it was given, and the call
    flags ERR_WRITE_SLOT."""
    case, bt, slots, k_new, v_new, row0, plan, spare = _frame("small")
    cfg = case.config
    moved = slots.clone()
    moved[row0 + 300] = spare  # a chunk token sent to a slot no table holds
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    kernels.paged_prefill(case.q, case.k_cache, case.v_cache, bt, case.cu_seqlens_q, case.q_start, 256,
                          cfg.block_size, cfg.scale, err_flags=err, new_kv=(k_new, v_new, moved), src_row0=row0)
    torch.cuda.synchronize()
    assert err.item() & ERR_WRITE_SLOT
    assert torch.equal(case.k_cache[spare], k_new[row0 + 300])


def test_fused_write_flags_a_bad_block_id_of_a_new_token():
    """A chunk with no cached prefix whose block table holds an id outside the
    pool: its new keys are read from the given rows (no block id is looked up
    for them), and the check after the walk flags the bad id."""
    from infrared_amd._lib import ERR_BLOCK_RANGE

    case, bt, slots, k_new, v_new, row0, plan, _ = _frame("small")
    cfg = case.config
    assert CASES["small"][1][0] == 0  # sequence 0: all its keys new
    bad_bt = bt.clone()
    bad_bt[0, 3] = case.k_cache.shape[0] // cfg.block_size + 5
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    kernels.paged_prefill(case.q, case.k_cache, case.v_cache, bad_bt, case.cu_seqlens_q, case.q_start, 256,
                          cfg.block_size, cfg.scale, err_flags=err, new_kv=(k_new, v_new, slots), src_row0=row0)
    torch.cuda.synchronize()
    assert err.item() & ERR_BLOCK_RANGE


def test_fused_write_refuses_rows_outside_the_written_range():
    case, bt, slots, k_new, v_new, row0, plan, _ = _frame("small")
    cfg = case.config
    with pytest.raises(RuntimeError, match="must lie within"):
        kernels.paged_prefill(case.q, case.k_cache, case.v_cache, bt, case.cu_seqlens_q, case.q_start, 256,
                              cfg.block_size, cfg.scale, new_kv=(k_new, v_new, slots), src_row0=row0 + 1)
