"""Host-side logic of the product (no GPU): bucketing, static decode inputs and
the vectorised metadata builders, against the reference tests' known answers
and the oracle's loop restatements."""

from __future__ import annotations

import pytest
import torch

from infrared_amd import hip_graph, metadata
from oracle import naive as O


def test_default_buckets_kat(golden):
    for n, want in golden["default_buckets"]["cases"]:
        assert hip_graph.default_buckets(n) == tuple(want)
    with pytest.raises(ValueError, match="max_num_seqs"):
        hip_graph.default_buckets(0)


def test_pick_bucket_kat(golden):
    kat = golden["pick_bucket"]
    for b, want in kat["cases"]:
        assert hip_graph.pick_bucket(b, tuple(kat["buckets"])) == want
    with pytest.raises(ValueError, match="exceeds largest bucket"):
        hip_graph.pick_bucket(kat["rejects"][0], tuple(kat["buckets"]))


def test_build_static_inputs_real_rows(golden):
    kat = golden["decode_static_inputs"]
    inp = hip_graph.build_decode_static_inputs(
        kat["block_tables"], kat["num_cached"], kat["last_tokens"], kat["bucket_b"], kat["t_max"],
        kat["block_size"], "cpu", torch.float32,
    )
    b, t = kat["bucket_b"], kat["t_max"]
    assert inp.ids.shape == (b, 1) and inp.positions.shape == (b, 1)
    assert inp.write_slots.shape == (b,) and inp.gather_slots.shape == (b, t)
    assert inp.mask.shape == (b, 1, 1, t)
    e = kat["expect"]
    assert inp.positions[0, 0].item() == e["positions_row0"]
    assert inp.write_slots[0].item() == e["write_slots_row0"]
    assert inp.ids[0, 0].item() == e["ids_row0"]
    assert inp.write_slots[1].item() == e["write_slots_row1"]
    neg = torch.finfo(torch.float32).min
    for i, n in enumerate(e["mask_valid_len"]):
        assert (inp.mask[i, 0, 0, :n] == 0).all() and (inp.mask[i, 0, 0, n:] == neg).all()
        assert inp.context_lens[i].item() == n
    # the full gather rows equal the oracle's loop construction
    ctx = [n + 1 for n in kat["num_cached"]]
    ref = O.decode_gather_slots(kat["block_tables"], ctx, kat["block_size"], t)
    assert torch.equal(inp.gather_slots[:2], ref)


def test_build_static_inputs_pads_by_repeating_row_zero(golden):
    kat = golden["decode_static_pad_by_repeat"]
    inp = hip_graph.build_decode_static_inputs(
        kat["block_tables"], kat["num_cached"], kat["last_tokens"], kat["bucket_b"], kat["t_max"],
        kat["block_size"], "cpu", torch.float32,
    )
    for pad in kat["padded_rows"]:
        for name in ("ids", "positions", "write_slots", "gather_slots", "mask", "block_tables", "context_lens"):
            assert torch.equal(getattr(inp, name)[pad], getattr(inp, name)[0]), name


def test_build_static_inputs_rejects_overlong_context(golden):
    kat = golden["decode_static_overlong"]
    with pytest.raises(ValueError, match=kat["error"]):
        hip_graph.build_decode_static_inputs(
            kat["block_tables"], kat["num_cached"], kat["last_tokens"], kat["bucket_b"],
            kat["t_max"], kat["block_size"], "cpu", torch.float32,
        )
    with pytest.raises(ValueError, match="bucket_b"):
        hip_graph.build_decode_static_inputs([[0]], [0], [1, 2], 1, 8, 8, "cpu", torch.float32)


def test_graph_shaped_metadata_matches_tight(golden):
    """Padding the bucket and the key axis leaves the real rows' metadata unchanged
    (the metadata half of tests/test_cuda_graph.py:178-210)."""
    kat = golden["graph_shaped_forward"]
    args = (kat["block_tables"], kat["num_cached"], [7, 11])
    tight = hip_graph.build_decode_static_inputs(
        *args, kat["tight"]["bucket_b"], kat["tight"]["t_max"], kat["block_size"], "cpu", torch.float32
    )
    pad = hip_graph.build_decode_static_inputs(
        *args, kat["padded"]["bucket_b"], kat["padded"]["t_max"], kat["block_size"], "cpu", torch.float32
    )
    assert tight.write_slots.tolist() == kat["write_slots"]
    assert torch.equal(pad.write_slots[:2], tight.write_slots)
    assert torch.equal(pad.context_lens[:2], tight.context_lens)
    t = kat["tight"]["t_max"]
    assert torch.equal(pad.gather_slots[:2, :t], tight.gather_slots)
    assert pad.gather_slots[:2, t:].eq(0).all()


def test_blocks_for_kat(golden):
    kat = golden["blocks_for"]
    for n, want in kat["cases"]:
        assert metadata.blocks_for(n, kat["block_size"]) == want


@pytest.mark.parametrize("bs", [1, 4, 16, 32])
def test_gather_slots_from_tables_matches_loop(bs):
    g = torch.Generator().manual_seed(bs)
    b = 6
    ctx = torch.randint(1, 90, (b,), generator=g)
    nblk = (ctx + bs - 1) // bs
    perm = torch.randperm(int(nblk.sum()) + 5, generator=g)
    tables, off = [], 0
    for n in nblk.tolist():
        tables.append(perm[off : off + n].tolist())
        off += n
    bt = metadata.block_tables_tensor(tables, "cpu")
    t_max = int(ctx.max()) + 3
    got = metadata.gather_slots_from_tables(bt, ctx.to(torch.int32), bs, t_max)
    assert torch.equal(got, O.decode_gather_slots(tables, ctx.tolist(), bs, t_max))
    nc = ctx - 1
    ws = metadata.decode_write_slots(bt, nc, bs)
    assert ws.tolist() == [O.slot(tables[i], int(nc[i]), bs) for i in range(b)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_decode_mask_matches_oracle(dtype):
    ctx = [1, 5, 17, 3]
    got = metadata.decode_mask(torch.tensor(ctx, dtype=torch.int32), 20, dtype)
    assert torch.equal(got, O.decode_mask(ctx, 20, dtype))


@pytest.mark.parametrize("bs", [1, 5, 16])
def test_packed_write_slots_match_the_slot_loop(bs):
    """The vectorised write slots of a packed step (prefill chunks after cached
    prefixes, decode rows as one-token chunks, an empty chunk) equal the
    reference engine's per-token loop slot(bt, p) over each chunk's positions
    (infrared/engine/paged_engine.py:481-494, :621-625)."""
    g = torch.Generator().manual_seed(bs)
    num_cached = [0, 37, 5, 120, 9]
    q_lens = [23, 1, 0, 40, 1]
    tables = []
    for c, n in zip(num_cached, q_lens):
        nb = metadata.blocks_for(c + n, bs) + 2
        tables.append(torch.randint(0, 10_000, (nb,), generator=g).tolist())
    bt = metadata.block_tables_tensor(tables, "cpu")
    got = metadata.packed_write_slots(bt, torch.tensor(num_cached), torch.tensor(q_lens), bs)
    want = [O.slot(t, p, bs) for t, c, n in zip(tables, num_cached, q_lens) for p in range(c, c + n)]
    assert got.dtype == torch.int64 and got.tolist() == want


def test_block_tables_tensor_pads_with_block_zero():
    bt = metadata.block_tables_tensor([[5, 6, 7], [], [9]], "cpu", 4)
    assert bt.dtype == torch.int32 and bt.tolist() == [[5, 6, 7, 0], [0, 0, 0, 0], [9, 0, 0, 0]]
    with pytest.raises(ValueError, match="longer than width"):
        metadata.block_tables_tensor([[1, 2, 3]], "cpu", 2)


def test_prefill_plan_pays_for_long_contexts_on_any_grid():
    """A call whose longest context exceeds PLAN_CUT_KEYS is planned whatever
    its workgroup count (decided before the device is asked for its CUs)."""
    from infrared_amd import kernels

    keys = kernels.PLAN_CUT_KEYS
    assert kernels.prefill_plan_pays(1, 200, 28, 4, "cpu", max_keys=keys + 1)
    assert not kernels.prefill_plan_pays(0, 200, 28, 4, "cpu", max_keys=keys + 1)  # nothing to plan
    assert not kernels.prefill_plan_pays(1, 200, 28, 5, "cpu", max_keys=keys + 1)  # heads not grouped
    assert kernels.prefill_plan_pays(1, 200, 28, 4, "cpu", max_keys=keys + 1, dtype=torch.float32)
    # fp32 groups wider than its kernel's 64 columns are refused, not planned
    assert not kernels.prefill_plan_pays(1, 200, 65, 1, "cpu", max_keys=keys + 1, dtype=torch.float32)


def test_seam_folds_the_write_only_for_rows_the_prefill_kernel_can_take():
    """The seam hands the step's rows to the prefill launch only for this
    package's pool, 16-bit rows of the pool's dtype in 16-byte pieces and
    int64 write slots; anything else is written by pool.write first."""
    from infrared_amd.paged_attention import _fusable

    class Pool:  # the attributes the check reads
        def __init__(self, dtype):
            self.k = torch.zeros(2, 64, 4, 128, dtype=dtype)

        def reference_varlen_form(self):  # pragma: no cover - presence is what counts
            pass

    k = torch.zeros(10, 4, 128, dtype=torch.bfloat16)
    v = torch.zeros_like(k)
    slots = torch.arange(10, dtype=torch.int64)
    pool = Pool(torch.bfloat16)
    assert _fusable(pool, 1, (k, v, slots))
    assert not _fusable(pool, 1, (k, v, None))
    assert not _fusable(pool, 1, (k, v, slots.int()))
    assert not _fusable(pool, 1, (k, v, slots[:9]))
    assert not _fusable(pool, 1, (k.float(), v.float(), slots))
    assert not _fusable(Pool(torch.float32), 1, (k.float(), v.float(), slots))
    wide = torch.zeros(10, 4, 130, dtype=torch.bfloat16)[..., :128]  # rows 260 elements apart
    assert not _fusable(pool, 1, (wide, wide, slots))
    shifted = torch.zeros(10 * 512 + 1, dtype=torch.bfloat16)[1:].view(10, 4, 128)  # 2-byte aligned
    assert not _fusable(pool, 1, (shifted, shifted, slots))

    class ForeignPool:  # a pool without this package's kernels
        k = pool.k

    assert not _fusable(ForeignPool(), 1, (k, v, slots))


def test_record_wait_returns_once_the_tag_is_there():
    """A device-written host record already carrying the call's tag is read at
    once: no poll runs out and the stream is never synchronised (which needs a
    device, absent here)."""
    import numpy as np

    from infrared_amd import kernels

    host = np.zeros(16, dtype=np.int32)
    host[7] = 12345
    kernels.await_record(host, 7, 12345, torch.device("cuda"))
