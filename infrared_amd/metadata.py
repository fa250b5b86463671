"""Device-side paged metadata builders (the engine side of the seam).

The reference engine builds per-step metadata with Python loops and one
host->device copy per sequence (``infrared/engine/paged_engine.py:303-314``,
``infrared/engine/cuda_graph.py:137-148``). These builders produce the same
tensors vectorised, plus the ``block_tables``/``context_lens`` pair the HIP
decode kernel reads, so a caller fills ``PagedContext`` directly:

- ``slot(bt, p, bs) = bt[p // bs] * bs + p % bs`` (``paged_engine.py:621-625``);
- ``gather_slots[i, p] = slot(bt_i, p)`` for ``p < ctx_i``, ``0`` after
  (``paged_engine.py:306-314``);
- decode mask ``0`` for ``col < ctx_i``, ``finfo(dtype).min`` after
  (``paged_engine.py:630-638``);
- packed prefill / mixed steps (``paged_engine.py:194-207``, ``:461-516``):
  ``write_slots`` of every new token in packing order, ``cu_seqlens_q`` /
  ``q_start`` for the prefill kernel and, on request, the reference's packed
  ``gather_slots`` + varlen mask (``infrared/model/inputs.py:57-85``).
"""

from __future__ import annotations

from collections.abc import Sequence

import numpy as np
import torch

from infrared_amd.paged_kv_cache import PagedContext, PagedKVPool, row_split


def slot(block_table: Sequence[int], pos: int, block_size: int) -> int:
    """Flat physical slot of logical position ``pos``."""
    return block_table[pos // block_size] * block_size + (pos % block_size)


def blocks_for(num_tokens: int, block_size: int) -> int:
    """Blocks ``num_tokens`` tokens occupy (ceil divide; ``block_manager.py:82-84``)."""
    return (num_tokens + block_size - 1) // block_size


def block_tables_tensor(
    block_tables: Sequence[Sequence[int]], device: torch.device | str, width: int | None = None
) -> torch.Tensor:
    """``[B, width]`` int32, rows right-padded with block 0 (entries past a row's
    context are never read). Rows are copied whole into one host array (one
    copy per row, not per block id) and moved to the device at once."""
    lens = [len(r) for r in block_tables]
    w = max(lens, default=0) if width is None else width
    if any(n > w for n in lens):
        raise ValueError(f"a block table is longer than width {w}")
    arr = np.zeros((len(lens), w), dtype=np.int32)
    for i, (r, n) in enumerate(zip(block_tables, lens)):
        if n:
            arr[i, :n] = r
    return torch.from_numpy(arr).to(device)


def packed_write_slots(
    block_tables: torch.Tensor, num_cached: torch.Tensor, q_lens: torch.Tensor, block_size: int
) -> torch.Tensor:
    """``[sum(q_lens)]`` int64 slots of a packed step's new tokens, in packing
    order: sequence ``b``'s ``q_lens[b]`` tokens at positions ``num_cached[b] ..``
    map to ``slot(bt_b, p) = bt_b[p // bs] * bs + p % bs``
    (``infrared/engine/paged_engine.py:621-625``), computed on the tables' device."""
    dev = block_tables.device
    q_lens = q_lens.to(device=dev, dtype=torch.long)
    nc = num_cached.to(device=dev, dtype=torch.long)
    seq = torch.repeat_interleave(torch.arange(q_lens.numel(), device=dev), q_lens)
    first = torch.cumsum(q_lens, 0) - q_lens  # packed row of each sequence's first token
    pos = nc[seq] + (torch.arange(seq.numel(), device=dev) - first[seq])
    blk = block_tables.long()[seq, pos // block_size]
    return blk * block_size + pos % block_size


def gather_slots_from_tables(
    block_tables: torch.Tensor, context_lens: torch.Tensor, block_size: int, t_max: int
) -> torch.Tensor:
    """``[B, t_max]`` int64 slot ids of each row's history; ``0`` past ``context_lens``."""
    pos = torch.arange(t_max, device=block_tables.device)
    blk = torch.clamp(pos // block_size, max=max(block_tables.shape[1] - 1, 0))
    ids = block_tables.long().index_select(1, blk) if block_tables.shape[1] else torch.zeros(
        block_tables.shape[0], t_max, dtype=torch.long, device=block_tables.device
    )
    slots = ids * block_size + (pos % block_size)
    valid = pos[None, :] < context_lens.long()[:, None]
    return torch.where(valid, slots, torch.zeros_like(slots))


def decode_mask(
    context_lens: torch.Tensor, max_len: int, dtype: torch.dtype
) -> torch.Tensor:
    """Additive ``[B, 1, 1, max_len]``: 0 for ``col < ctx``, ``finfo(dtype).min`` after."""
    cols = torch.arange(max_len, device=context_lens.device)
    invalid = cols[None, :] >= context_lens.long()[:, None]
    mask = torch.zeros(context_lens.shape[0], 1, 1, max_len, dtype=dtype, device=context_lens.device)
    return mask.masked_fill(invalid[:, None, None, :], torch.finfo(dtype).min)


def decode_write_slots(
    block_tables: torch.Tensor, num_cached: torch.Tensor, block_size: int
) -> torch.Tensor:
    """``[B]`` int64 slot of each sequence's new token (position ``num_cached``)."""
    nc = num_cached.long()
    blk = (nc // block_size)[:, None]
    ids = torch.gather(block_tables.long(), 1, blk)[:, 0]
    return ids * block_size + nc % block_size


def decode_context(
    pool: PagedKVPool,
    block_tables: Sequence[Sequence[int]],
    num_cached: Sequence[int],
    *,
    t_max: int | None = None,
    use_triton: bool = True,
    mask_dtype: torch.dtype | None = None,
) -> tuple[PagedContext, torch.Tensor]:
    """One batched decode step's ``PagedContext`` + mask, as ``_decode_logits_eager``
    builds them (``infrared/engine/paged_engine.py:290-332``) plus the block-table fields.

    Each sequence's new token sits at position ``num_cached[i]`` and attends
    ``[0, num_cached[i]]`` (``context_len = num_cached + 1``).
    """
    dev = pool.device
    bs = pool.block_size
    ctx = [n + 1 for n in num_cached]
    width = max(blocks_for(c, bs) for c in ctx)
    bt = block_tables_tensor([list(r)[:width] for r in block_tables], dev, width)
    cl = torch.tensor(ctx, dtype=torch.int32, device=dev)
    t = max(ctx) if t_max is None else t_max
    gs = gather_slots_from_tables(bt, cl, bs, t)
    ws = decode_write_slots(bt, torch.tensor(list(num_cached), device=dev), bs)
    mask = decode_mask(cl, t, mask_dtype or pool.dtype)
    return PagedContext(pool, ws, gs, use_triton, bt, cl), mask


def prefill_context(
    pool: PagedKVPool,
    block_tables: Sequence[Sequence[int]],
    num_cached: Sequence[int],
    q_lens: Sequence[int],
    *,
    use_triton: bool = True,
    with_mask: bool = False,
    mask_dtype: torch.dtype | None = None,
) -> tuple[PagedContext, torch.Tensor | None]:
    """``PagedContext`` of one packed step: sequence ``i`` forwards ``q_lens[i]``
    new tokens at positions ``num_cached[i] ..``, packed in sequence order into
    one ``B = 1`` frame (a decode row is ``q_len = 1``).

    ``with_mask`` also builds the reference's packed metadata -- ``gather_slots``
    ``[1, K]`` over the union of the sequences' keys and the varlen mask
    ``[1, 1, Q, K]`` -- for the gather_slots + mask kernel
    (``use_triton=False``) or the reference-form path; it is quadratic in the
    step size.
    """
    dev = pool.device
    bs = pool.block_size
    if not (len(block_tables) == len(num_cached) == len(q_lens)):
        raise ValueError("block_tables, num_cached and q_lens must have one entry per sequence")
    lengths = [c + n for c, n in zip(num_cached, q_lens)]
    width = max(blocks_for(n, bs) for n in lengths) if lengths else 0
    rows = [r[: max(width, 1)] for r in block_tables]
    bt = block_tables_tensor(rows, dev, width)
    meta = torch.tensor([list(num_cached), list(q_lens)], dtype=torch.int32).to(dev)  # one host->device copy
    nc_t, ql_t = meta[0], meta[1]
    cu = torch.zeros(len(q_lens) + 1, dtype=torch.int32, device=dev)
    cu[1:] = torch.cumsum(ql_t, 0)
    ctx = PagedContext(
        pool,
        packed_write_slots(bt, nc_t, ql_t, bs),
        None,
        use_triton,
        bt,
        None,
        cu,
        nc_t.contiguous(),
        max(q_lens, default=0),
    )
    ctx.row_split = row_split(bt, num_cached, q_lens)
    if not with_mask:
        return ctx, None
    k_seq, k_pos, gslots = [], [], []
    for i, (r, n) in enumerate(zip(rows, lengths)):
        for p in range(n):
            k_seq.append(i)
            k_pos.append(p)
            gslots.append(slot(r, p, bs))
    q_seq = torch.tensor([i for i, n in enumerate(q_lens) for _ in range(n)], device=dev)
    q_pos = torch.tensor([c + j for c, n in zip(num_cached, q_lens) for j in range(n)], device=dev)
    k_seq_t = torch.tensor(k_seq, device=dev)
    k_pos_t = torch.tensor(k_pos, device=dev)
    allowed = (q_seq[:, None] == k_seq_t[None, :]) & (k_pos_t[None, :] <= q_pos[:, None])
    dtype = mask_dtype or pool.dtype
    mask = torch.zeros(1, 1, len(q_seq), len(k_seq), dtype=dtype, device=dev)
    mask = mask.masked_fill(~allowed[None, None], torch.finfo(dtype).min)
    ctx.gather_slots = torch.tensor([gslots], dtype=torch.int64, device=dev)
    return ctx, mask
