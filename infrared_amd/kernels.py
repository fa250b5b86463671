"""Tensor-level wrappers of the C ABI: validate shapes on the host, pass raw
pointers and torch's current stream, raise ``RuntimeError`` on any failure.

Each wrapper launches asynchronously and allocates at most its output (and
the decode workspace when one is not supplied), so it can run under hipGraph
capture.
"""

from __future__ import annotations

import itertools
from dataclasses import dataclass

import torch

from infrared_amd._lib import check, dtype_code, lib, ptr, require_device, stream_ptr


def _last_dim_contiguous(name: str, t: torch.Tensor) -> None:
    if t.stride(-1) != 1:
        raise RuntimeError(f"{name}: the last (head_dim) dimension must be contiguous")


def _cache_layer(name: str, cache: torch.Tensor) -> None:
    if cache.dim() != 3:
        raise RuntimeError(f"{name}: expected one pool layer [num_slots, num_kv_heads, head_dim]")
    _last_dim_contiguous(name, cache)


def kv_scatter(
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    slots: torch.Tensor,
    err_flags: torch.Tensor | None = None,
) -> None:
    """``k_cache[slots] = k; v_cache[slots] = v`` (``PagedKVPool.write`` semantics).

    ``k``/``v``: ``[N, H_kv, D]``; ``slots``: ``[N]`` int64. Negative slots are
    skipped (padding sentinel); slots ``>= num_slots`` are skipped and flagged.
    """
    dev = require_device(k_cache, v_cache, k, v, slots)
    _cache_layer("kv_scatter", k_cache)
    if v_cache.shape != k_cache.shape or v_cache.stride() != k_cache.stride():
        raise RuntimeError("kv_scatter: k_cache and v_cache must have the same shape and strides")
    n, h, d = k.shape
    if v.shape != k.shape or (h, d) != tuple(k_cache.shape[1:]):
        raise RuntimeError(
            f"kv_scatter: k {tuple(k.shape)} / v {tuple(v.shape)} do not match pool rows "
            f"{tuple(k_cache.shape[1:])}"
        )
    if k.dtype != k_cache.dtype or v.dtype != k_cache.dtype:
        raise RuntimeError(f"kv_scatter: dtype mismatch ({k.dtype}, {v.dtype} vs pool {k_cache.dtype})")
    if slots.dtype != torch.int64 or slots.shape != (n,):
        raise RuntimeError(f"kv_scatter: slots must be int64 [{n}], got {slots.dtype} {tuple(slots.shape)}")
    _last_dim_contiguous("kv_scatter k", k)
    _last_dim_contiguous("kv_scatter v", v)
    slots = slots.contiguous()
    rc = lib().ir_kv_scatter(
        ptr(k), k.stride(0), k.stride(1), ptr(v), v.stride(0), v.stride(1),
        ptr(k_cache), ptr(v_cache), k_cache.stride(0), k_cache.stride(1), k_cache.shape[0],
        ptr(slots), n, h, d, dtype_code(k_cache.dtype), ptr(err_flags), stream_ptr(dev),
    )
    check(rc, "ir_kv_scatter")


def gather_slots(
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    slots: torch.Tensor,
    err_flags: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """``(k_cache[slots], v_cache[slots])`` for any-shaped int64 ``slots`` -> ``[*slots.shape, H, D]``."""
    dev = require_device(k_cache, v_cache, slots)
    _cache_layer("gather_slots", k_cache)
    if slots.dtype != torch.int64:
        raise RuntimeError("gather_slots: slots must be int64")
    flat = slots.reshape(-1).contiguous()
    h, d = k_cache.shape[1:]
    out_k = torch.empty(flat.numel(), h, d, dtype=k_cache.dtype, device=dev)
    out_v = torch.empty_like(out_k)
    rc = lib().ir_gather_slots(
        ptr(k_cache), ptr(v_cache), k_cache.stride(0), k_cache.stride(1), k_cache.shape[0],
        ptr(flat), flat.numel(), h, d, dtype_code(k_cache.dtype), ptr(out_k), ptr(out_v),
        ptr(err_flags), stream_ptr(dev),
    )
    check(rc, "ir_gather_slots")
    return out_k.reshape(*slots.shape, h, d), out_v.reshape(*slots.shape, h, d)


def paged_gather(
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    block_size: int,
    max_ctx: int,
    err_flags: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Dense ``[B, max_ctx, H_kv, D]`` K/V histories through the block tables (zero-padded)."""
    dev = require_device(k_cache, v_cache, block_tables, context_lens)
    _cache_layer("paged_gather", k_cache)
    _check_tables("paged_gather", block_tables, context_lens)
    b = block_tables.shape[0]
    h, d = k_cache.shape[1:]
    out_k = torch.empty(b, max_ctx, h, d, dtype=k_cache.dtype, device=dev)
    out_v = torch.empty_like(out_k)
    num_blocks = k_cache.shape[0] // block_size
    rc = lib().ir_paged_gather(
        ptr(k_cache), ptr(v_cache), k_cache.stride(0), k_cache.stride(1), num_blocks, block_size,
        ptr(block_tables), block_tables.stride(0), block_tables.shape[1], ptr(context_lens), b,
        max_ctx, h, d, dtype_code(k_cache.dtype), ptr(out_k), ptr(out_v), ptr(err_flags),
        stream_ptr(dev),
    )
    check(rc, "ir_paged_gather")
    return out_k, out_v


def _check_tables(name: str, block_tables: torch.Tensor, context_lens: torch.Tensor) -> None:
    if block_tables.dtype != torch.int32 or block_tables.dim() != 2 or block_tables.stride(1) != 1:
        raise RuntimeError(f"{name}: block_tables must be int32 [B, max_blocks] with contiguous rows")
    if context_lens.dtype != torch.int32 or context_lens.shape != (block_tables.shape[0],):
        raise RuntimeError(f"{name}: context_lens must be int32 [B]")
    if not context_lens.is_contiguous():
        raise RuntimeError(f"{name}: context_lens must be contiguous")


def decode_workspace_bytes(
    num_seqs: int, num_q_heads: int, num_kv_heads: int, head_dim: int, max_blocks: int,
    block_size: int, partition_tokens: int = 0,
) -> int:
    return int(lib().ir_paged_decode_workspace_size(
        num_seqs, num_q_heads, num_kv_heads, head_dim, max_blocks, block_size, partition_tokens
    ))


def decode_num_counters(num_seqs: int, num_q_heads: int, num_kv_heads: int) -> int:
    """int32 arrival counters a split decode needs (zero at rest; one buffer serves every shape)."""
    return int(lib().ir_paged_decode_num_counters(num_seqs, num_q_heads, num_kv_heads))


def _counters_for(counters: torch.Tensor | None, n: int, dev) -> torch.Tensor:
    if counters is None:
        return torch.zeros(max(n, 1), dtype=torch.int32, device=dev)
    if counters.dtype != torch.int32 or not counters.is_contiguous() or counters.numel() < n:
        raise RuntimeError(f"decode counters must be a contiguous int32 tensor of >= {n} zeros")
    return counters


def default_partition(num_seqs: int, num_kv_heads: int, max_blocks: int, block_size: int) -> int:
    return int(lib().ir_paged_decode_default_partition(num_seqs, num_kv_heads, max_blocks, block_size))


def paged_decode(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    block_size: int,
    scale: float,
    out: torch.Tensor | None = None,
    partition_tokens: int = 0,
    workspace: torch.Tensor | None = None,
    err_flags: torch.Tensor | None = None,
    counters: torch.Tensor | None = None,
) -> torch.Tensor:
    """GQA paged decode: ``q`` ``[B, H_q, D]`` -> ``[B, H_q, D]``.

    ``block_tables`` int32 ``[B, max_blocks]``, ``context_lens`` int32 ``[B]``.
    ``workspace`` (uint8 scratch, 256-byte aligned) and ``counters`` (int32,
    zero-filled before first use; every call leaves them at zero) are allocated
    when not given and the longest possible context needs more than one
    partition.
    """
    dev = require_device(q, k_cache, v_cache, block_tables, context_lens)
    _cache_layer("paged_decode", k_cache)
    _check_tables("paged_decode", block_tables, context_lens)
    if q.dim() != 3:
        raise RuntimeError(f"paged_decode: q must be [B, H_q, D], got {tuple(q.shape)}")
    b, hq, d = q.shape
    h_kv = k_cache.shape[1]
    if d != k_cache.shape[2] or q.dtype != k_cache.dtype or v_cache.shape != k_cache.shape:
        raise RuntimeError("paged_decode: q / pool shape or dtype mismatch")
    if block_tables.shape[0] != b:
        raise RuntimeError("paged_decode: block_tables rows != batch")
    _last_dim_contiguous("paged_decode q", q)
    if out is None:
        out = torch.empty(b, hq, d, dtype=q.dtype, device=dev)
    max_blocks = block_tables.shape[1]
    if partition_tokens <= 0:
        partition_tokens = default_partition(b, h_kv, max_blocks, block_size)
    need = decode_workspace_bytes(b, hq, h_kv, d, max_blocks, block_size, partition_tokens)
    n_ctr = 0
    if need > 0:
        if workspace is None or workspace.numel() < need:
            workspace = torch.empty(need, dtype=torch.uint8, device=dev)
        n_ctr = decode_num_counters(b, hq, h_kv)
        counters = _counters_for(counters, n_ctr, dev)
    rc = lib().ir_paged_decode(
        ptr(q), q.stride(0), q.stride(1), ptr(k_cache), ptr(v_cache), k_cache.stride(0),
        k_cache.stride(1), k_cache.shape[0] // block_size, block_size, ptr(block_tables),
        block_tables.stride(0), max_blocks, ptr(context_lens), ptr(out), out.stride(0),
        out.stride(1), b, hq, h_kv, d, float(scale), dtype_code(q.dtype), partition_tokens,
        ptr(counters) if need > 0 else None, n_ctr, ptr(workspace) if need > 0 else None, need,
        ptr(err_flags), stream_ptr(dev),
    )
    check(rc, "ir_paged_decode")
    return out


@dataclass(frozen=True)
class DecodePlan:
    """A decode plan (``ir_paged_decode_plan``) and the shape it was built for.

    ``buf`` holds the schedule of one batch of decode metadata; every layer of
    the step runs on it with :func:`paged_decode_planned`. Rebuild it (same or
    new buffer) when ``block_tables``/``context_lens`` change, after the runs
    that read it.
    """

    buf: torch.Tensor
    num_seqs: int
    num_q_heads: int
    num_kv_heads: int
    max_blocks: int
    block_size: int
    num_blocks: int
    slot_stride: int
    head_stride: int
    dtype: torch.dtype
    share_groups: bool = False


def decode_plan_bytes(num_seqs: int, num_q_heads: int, num_kv_heads: int, max_blocks: int, block_size: int) -> int:
    """Plan bytes for this shape; 0 when it is not plannable (then use :func:`paged_decode`)."""
    return int(lib().ir_paged_decode_plan_bytes(num_seqs, num_q_heads, num_kv_heads, max_blocks, block_size))


_CU_COUNT: dict[int, int] = {}


def decode_plan_pays(num_seqs: int, num_q_heads: int, num_kv_heads: int, max_blocks: int, block_size: int,
                     device: torch.device | str | int | None = None) -> bool:
    """Whether the planned schedule is the faster decode for this shape: it is
    plannable, and either the batch has a unit (sequence x KV head x group of
    <= 16 query heads) per CU or its block tables can hold 16 tiles (256 keys)
    per CU across the units. Below that the work is too small to spread: the
    plan's per-call overhead outweighs the balance, and :func:`paged_decode`'s
    fixed split-KV partitions win. Measured on MI355X (28 q / 4 kv heads, bf16,
    per call): 64 sequences 57.2 (fixed) vs 49.7 us; 8 of 2k..32k keys 72.0 vs
    55.0 us; 16 skewed long ones 33.4 vs 31.8 us; 16 of 16..1024 keys 16.3 vs
    11.6 us; but 8 fp32 sequences of <= 512 keys 7.1 vs 10.5 us and 16 of <= 300
    keys in tables of that width 7.9 vs 11.0 us."""
    if decode_plan_bytes(num_seqs, num_q_heads, num_kv_heads, max_blocks, block_size) <= 0:
        return False
    idx = torch.device(device if device is not None else "cuda").index
    idx = torch.cuda.current_device() if idx is None else idx
    if idx not in _CU_COUNT:
        _CU_COUNT[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    cus = _CU_COUNT[idx]
    units = num_seqs * num_kv_heads * ((num_q_heads // num_kv_heads + 15) // 16)
    tiles = units * ((max_blocks * block_size + 15) // 16)
    return units >= cus or tiles >= 16 * cus


def planned_workspace_bytes(num_seqs: int, num_q_heads: int, num_kv_heads: int, head_dim: int) -> int:
    return int(lib().ir_paged_decode_planned_workspace_bytes(num_seqs, num_q_heads, num_kv_heads, head_dim))


def decode_plan(
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    num_q_heads: int,
    k_cache: torch.Tensor,
    block_size: int,
    buf: torch.Tensor | None = None,
    err_flags: torch.Tensor | None = None,
    share_groups: bool = False,
) -> DecodePlan:
    """Builds the balanced decode schedule of ``(block_tables, context_lens)``
    for query heads ``num_q_heads`` over pool layers shaped like ``k_cache``
    ``[num_slots, H_kv, D]`` (any layer: all share the strides).
    ``share_groups``: consecutive sequences whose tables begin with the same
    block ids (a shared cached prefix) run as pairs, one unit per KV head with
    both sequences' query heads, so the shared blocks are read once (taken when
    a KV head has at most 8 query heads)."""
    dev = require_device(block_tables, context_lens, k_cache)
    _cache_layer("decode_plan", k_cache)
    _check_tables("decode_plan", block_tables, context_lens)
    b, max_blocks = block_tables.shape
    h_kv = k_cache.shape[1]
    need = decode_plan_bytes(b, num_q_heads, h_kv, max_blocks, block_size)
    if need <= 0:
        raise RuntimeError(f"decode_plan: shape not plannable (batch {b}, block_size {block_size})")
    if buf is None or buf.numel() < need:
        buf = torch.empty(need, dtype=torch.uint8, device=dev)
    if buf.dtype != torch.uint8 or buf.data_ptr() % 256:
        raise RuntimeError("decode_plan: buf must be a 256-byte aligned uint8 tensor")
    rc = lib().ir_paged_decode_plan(
        ptr(block_tables), block_tables.stride(0), max_blocks, ptr(context_lens), b, num_q_heads, h_kv,
        block_size, k_cache.shape[0] // block_size, k_cache.stride(0), k_cache.stride(1),
        dtype_code(k_cache.dtype), PLAN_SHARE_GROUPS if share_groups else 0, ptr(buf), buf.numel(), ptr(err_flags),
        stream_ptr(dev),
    )
    check(rc, "ir_paged_decode_plan")
    return DecodePlan(buf, b, num_q_heads, h_kv, max_blocks, block_size, k_cache.shape[0] // block_size,
                      k_cache.stride(0), k_cache.stride(1), k_cache.dtype, bool(share_groups))


def paged_decode_planned(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    plan: DecodePlan,
    scale: float,
    out: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
    err_flags: torch.Tensor | None = None,
    counters: torch.Tensor | None = None,
) -> torch.Tensor:
    """:func:`paged_decode` over a plan: ``q`` ``[B, H_q, D]`` -> ``[B, H_q, D]``.
    ``workspace`` (uint8 scratch) and ``counters`` (int32 zeros, left at zero)
    are allocated when not given."""
    dev = require_device(q, k_cache, v_cache, plan.buf)
    _cache_layer("paged_decode_planned", k_cache)
    if q.dim() != 3:
        raise RuntimeError(f"paged_decode_planned: q must be [B, H_q, D], got {tuple(q.shape)}")
    b, hq, d = q.shape
    if (b, hq) != (plan.num_seqs, plan.num_q_heads) or k_cache.shape[1] != plan.num_kv_heads:
        raise RuntimeError("paged_decode_planned: q / pool heads differ from the plan's")
    if (k_cache.shape[0] // plan.block_size != plan.num_blocks or k_cache.stride(0) != plan.slot_stride
            or k_cache.stride(1) != plan.head_stride or k_cache.dtype != plan.dtype):
        raise RuntimeError("paged_decode_planned: pool layout differs from the plan's")
    if v_cache.shape != k_cache.shape or v_cache.stride() != k_cache.stride():
        raise RuntimeError("paged_decode_planned: v_cache must match k_cache's shape and strides")
    if d != k_cache.shape[2] or q.dtype != k_cache.dtype:
        raise RuntimeError("paged_decode_planned: q / pool shape or dtype mismatch")
    _last_dim_contiguous("paged_decode_planned q", q)
    if out is None:
        out = torch.empty(b, hq, d, dtype=q.dtype, device=dev)
    need = planned_workspace_bytes(b, hq, plan.num_kv_heads, d)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    n_ctr = decode_num_counters(b, hq, plan.num_kv_heads)
    counters = _counters_for(counters, n_ctr, dev)
    rc = lib().ir_paged_decode_planned(
        ptr(q), q.stride(0), q.stride(1), ptr(k_cache), ptr(v_cache), k_cache.stride(0), ptr(out),
        out.stride(0), out.stride(1), b, hq, plan.num_kv_heads, d, plan.max_blocks, plan.block_size,
        float(scale), dtype_code(q.dtype), PLAN_SHARE_GROUPS if plan.share_groups else 0, ptr(plan.buf),
        ptr(counters), n_ctr, ptr(workspace),
        workspace.numel(), ptr(err_flags), stream_ptr(dev),
    )
    check(rc, "ir_paged_decode_planned")
    return out


def paged_attention_masked(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    gather_slots: torch.Tensor,
    mask: torch.Tensor,
    scale: float,
    out: torch.Tensor | None = None,
    err_flags: torch.Tensor | None = None,
    run_if: torch.Tensor | None = None,
) -> torch.Tensor:
    """Attention over per-key slots + additive mask (the reference seam's metadata).

    ``q`` ``[B, Sq, H_q, D]``; ``gather_slots`` int64 ``[B, T]``; ``mask``
    broadcastable to ``[B, 1, Sq, T]``. Returns ``[B, Sq, H_q, D]``.
    ``run_if``: an int32 device flag; the kernel then writes ``out`` only
    when the flag is nonzero (read on the device, so it works under capture).
    """
    dev = require_device(q, k_cache, v_cache, gather_slots, mask)
    _cache_layer("paged_attention_masked", k_cache)
    if q.dim() != 4:
        raise RuntimeError(f"paged_attention_masked: q must be [B, Sq, H_q, D], got {tuple(q.shape)}")
    b, sq, hq, d = q.shape
    h_kv = k_cache.shape[1]
    if d != k_cache.shape[2] or q.dtype != k_cache.dtype:
        raise RuntimeError("paged_attention_masked: q / pool shape or dtype mismatch")
    if gather_slots.dtype != torch.int64 or gather_slots.dim() != 2 or gather_slots.shape[0] != b:
        raise RuntimeError("paged_attention_masked: gather_slots must be int64 [B, T]")
    t = gather_slots.shape[1]
    if mask.dim() != 4 or mask.shape[1] != 1:
        raise RuntimeError(f"paged_attention_masked: mask must be [B, 1, Sq, T], got {tuple(mask.shape)}")
    m = mask.expand(b, 1, sq, t)
    _last_dim_contiguous("paged_attention_masked q", q)
    if out is None:
        out = torch.empty(b, sq, hq, d, dtype=q.dtype, device=dev)
    if run_if is not None:
        require_device(q, run_if)
        if run_if.dtype != torch.int32 or run_if.numel() < 1:
            raise RuntimeError("paged_attention_masked: run_if must be an int32 device tensor")
    rc = lib().ir_paged_attention_masked(
        ptr(q), q.stride(0), q.stride(1), q.stride(2), ptr(k_cache), ptr(v_cache),
        k_cache.stride(0), k_cache.stride(1), k_cache.shape[0], ptr(gather_slots),
        gather_slots.stride(0), gather_slots.stride(1), ptr(m), m.stride(0), m.stride(2),
        m.stride(3), dtype_code(m.dtype), ptr(out), out.stride(0), out.stride(1), out.stride(2),
        b, sq, t, hq, h_kv, d, float(scale), dtype_code(q.dtype), ptr(err_flags), ptr(run_if), stream_ptr(dev),
    )
    check(rc, "ir_paged_attention_masked")
    return out


def rope_kv_scatter(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    slots: torch.Tensor,
    q_out: torch.Tensor | None = None,
    err_flags: torch.Tensor | None = None,
) -> torch.Tensor:
    """Rotary embedding of ``q`` (returned, ``[N, H_q, D]``) and ``k``, with the rotated
    ``k`` and ``v`` written into the pool layer at ``slots`` -- ``apply_rotary_pos_emb``
    followed by ``PagedKVPool.write`` in one launch, bit-identical to them.

    ``cos``/``sin``: fp32 ``[N, D]`` (``RotaryEmbedding`` output flattened over batch
    and sequence). ``q_out`` may be ``q`` itself (in place).
    """
    dev = require_device(q, k, v, cos, sin, k_cache, v_cache, slots)
    _cache_layer("rope_kv_scatter", k_cache)
    if q.dim() != 3 or k.dim() != 3 or v.shape != k.shape:
        raise RuntimeError("rope_kv_scatter: q [N, H_q, D], k and v [N, H_kv, D] expected")
    n, hq, d = q.shape
    if k.shape[0] != n or k.shape[2] != d or k.shape[1:] != k_cache.shape[1:]:
        raise RuntimeError("rope_kv_scatter: k/v rows do not match q or the pool")
    if q.dtype != k.dtype or k.dtype != k_cache.dtype or v.dtype != k.dtype:
        raise RuntimeError("rope_kv_scatter: dtype mismatch")
    if v_cache.stride() != k_cache.stride():
        raise RuntimeError("rope_kv_scatter: k_cache and v_cache must share strides")
    for name, t in (("cos", cos), ("sin", sin)):
        if t.dtype != torch.float32 or t.shape != (n, d) or t.stride(1) != 1:
            raise RuntimeError(f"rope_kv_scatter: {name} must be fp32 [N, D] with unit column stride")
    if cos.stride(0) != sin.stride(0):
        raise RuntimeError("rope_kv_scatter: cos and sin must share strides")
    if slots.dtype != torch.int64 or slots.shape != (n,):
        raise RuntimeError("rope_kv_scatter: slots must be int64 [N]")
    for name, t in (("q", q), ("k", k), ("v", v)):
        _last_dim_contiguous(f"rope_kv_scatter {name}", t)
    if q_out is None:
        q_out = torch.empty_like(q)
    rc = lib().ir_rope_kv_scatter(
        ptr(q), q.stride(0), q.stride(1), ptr(q_out), q_out.stride(0), q_out.stride(1), ptr(k), k.stride(0),
        k.stride(1), ptr(v), v.stride(0), v.stride(1), ptr(cos), ptr(sin), cos.stride(0), ptr(k_cache),
        ptr(v_cache), k_cache.stride(0), k_cache.stride(1), k_cache.shape[0], ptr(slots.contiguous()), n, hq,
        k.shape[1], d, dtype_code(q.dtype), ptr(err_flags), stream_ptr(dev),
    )
    check(rc, "ir_rope_kv_scatter")
    return q_out


PLAN_SHARE_GROUPS = 1  # IR_PLAN_SHARE_GROUPS
PLAN_F32 = 2  # IR_PLAN_F32


@dataclass(frozen=True)
class PrefillPlan:
    """A prefill work plan (``ir_paged_prefill_plan``) and the shape it was built
    for. ``buf`` holds the heaviest-first pieces of one step's prefill metadata
    plus their arrival counters and partial rows; every layer of the step runs
    on it with :func:`paged_prefill` (stream-ordered: the runs write into it).
    Rebuild it when ``cu_seqlens_q``/``q_start`` change. ``f32``: built for
    fp32 calls (``IR_PLAN_F32``: the fp32 kernel's 64-column items), which
    read only such a plan."""

    buf: torch.Tensor
    num_seqs: int
    max_q_len: int
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    f32: bool = False


def prefill_plan_bytes(num_seqs: int, max_q_len: int, num_q_heads: int, num_kv_heads: int, head_dim: int) -> int:
    """Bytes of a prefill plan for these shapes (0: nothing to plan)."""
    return int(lib().ir_paged_prefill_plan_bytes(num_seqs, max_q_len, num_q_heads, num_kv_heads, head_dim))


def prefill_plan_xcds() -> int:
    """XCDs the prefill plan places work on for the current device (1: one
    global heaviest-first order)."""
    return int(lib().ir_paged_prefill_plan_xcds())


PLAN_CUT_KEYS = 1024  # a call whose longest context exceeds this many keys is planned (its items get cut)


def prefill_plan_pays(num_seqs: int, max_q_len: int, num_q_heads: int, num_kv_heads: int,
                      device: torch.device | str | int | None = None, max_keys: int = 0,
                      dtype: torch.dtype = torch.bfloat16) -> bool:
    """Whether a plan can shorten the call: its workgroups outnumber the CUs,
    so the dispatch order -- and cutting the heaviest items -- decides which
    CU finishes last; or its longest context (``max_keys``, e.g. the block
    tables' width times the block size) exceeds ``PLAN_CUT_KEYS``, so cutting
    the long items into key ranges shortens the longest walk even when every
    workgroup starts at once (one 512-token chunk after 4,096 cached: 68 vs
    110 us; two 128-token chunks after 1,024: 26 vs 32 us). Otherwise every
    workgroup starts at once with nothing worth cutting. (Items are (sequence,
    block of 128 // n_rep query tokens), 4-wavefront workgroups; in fp32 blocks
    of 64 // n_rep tokens, two workgroups resident per CU, so an fp32 call is
    planned when its workgroups outnumber twice the CUs.)"""
    if num_seqs <= 0 or max_q_len <= 0 or num_kv_heads <= 0 or num_q_heads % num_kv_heads:
        return False
    n_rep = num_q_heads // num_kv_heads
    if dtype == torch.float32 and n_rep > 64:
        return False  # (the fp32 kernel refuses such groups)
    if max_keys > PLAN_CUT_KEYS:
        return True
    # workgroups resident at once: the 16-bit kernel's calls that fit one per
    # CU run a shape of their own, unplanned; the fp32 kernel holds two per CU
    per_cu = 1
    if dtype == torch.float32:
        tq, per_cu = 64 // n_rep, 2
    else:
        tq = (128 if n_rep <= 128 else 256) // n_rep
    idx = torch.device(device if device is not None else "cuda").index
    idx = torch.cuda.current_device() if idx is None else idx
    if idx not in _CU_COUNT:
        _CU_COUNT[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return num_seqs * -(-max_q_len // tq) * num_kv_heads > per_cu * _CU_COUNT[idx]


def prefill_plan(
    cu_seqlens_q: torch.Tensor,
    q_start: torch.Tensor,
    block_tables: torch.Tensor,
    total_q: int,
    max_q_len: int,
    block_size: int,
    num_q_heads: int,
    num_kv_heads: int,
    head_dim: int,
    buf: torch.Tensor | None = None,
    share_groups: bool = False,
    dtype: torch.dtype = torch.bfloat16,
) -> PrefillPlan:
    """Work plan of a prefill call's (sequence, query block) items, built on
    the device (``ir_paged_prefill_plan``); pass it to every layer's
    :func:`paged_prefill` over the same metadata. ``share_groups``: keep each
    (shared-prefix group, KV head) on one XCD -- groups are consecutive
    sequences whose ``block_tables`` (int32 ``[B, max_blocks]``) rows begin
    with the same block id -- so a shared prefix is fetched into one L2
    (fewer bytes from memory; slower on a prefill that has HBM to itself);
    by default one global heaviest-first order. Tables with other ids but the
    same shape run correctly on the plan. ``dtype``: the calls' dtype (fp32
    calls take a plan of their own kernel's items). ``buf`` (uint8, 256-byte
    aligned) is reused when large enough."""
    dev = require_device(cu_seqlens_q, q_start, block_tables)
    b = q_start.shape[0]
    f32 = dtype == torch.float32
    for name, t, n in (("cu_seqlens_q", cu_seqlens_q, b + 1), ("q_start", q_start, b)):
        if t.dtype != torch.int32 or t.shape != (n,) or not t.is_contiguous():
            raise RuntimeError(f"prefill_plan: {name} must be contiguous int32 [{n}]")
    if (block_tables.dtype != torch.int32 or block_tables.dim() != 2 or block_tables.shape[0] != b
            or block_tables.stride(1) != 1):
        raise RuntimeError(f"prefill_plan: block_tables must be int32 [{b}, max_blocks] with unit column stride")
    n = prefill_plan_bytes(b, max_q_len, num_q_heads, num_kv_heads, head_dim)
    if n <= 0:
        raise RuntimeError("prefill_plan: nothing to plan for these shapes")
    if buf is None or buf.numel() < n:
        buf = torch.empty(n, dtype=torch.uint8, device=dev)
    if buf.dtype != torch.uint8 or buf.data_ptr() % 256:
        raise RuntimeError("prefill_plan: buf must be a 256-byte aligned uint8 tensor")
    max_blocks = block_tables.shape[1]
    rc = lib().ir_paged_prefill_plan(
        ptr(cu_seqlens_q), ptr(q_start), ptr(block_tables), max(block_tables.stride(0), max_blocks), b,
        int(total_q), int(max_q_len), int(max_blocks), int(block_size), num_q_heads, num_kv_heads, head_dim,
        (PLAN_SHARE_GROUPS if share_groups else 0) | (PLAN_F32 if f32 else 0), ptr(buf), buf.numel(),
        stream_ptr(dev),
    )
    check(rc, "ir_paged_prefill_plan")
    return PrefillPlan(buf, b, int(max_q_len), num_q_heads, num_kv_heads, head_dim, f32)


def paged_prefill(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    q_start: torch.Tensor,
    max_q_len: int,
    block_size: int,
    scale: float,
    out: torch.Tensor | None = None,
    err_flags: torch.Tensor | None = None,
    plan: PrefillPlan | None = None,
    new_kv: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None,
    src_row0: int = 0,
) -> torch.Tensor:
    """Causal paged attention for packed query chunks: ``q`` ``[total_q, H_q, D]``.

    Sequence ``b`` owns rows ``cu_seqlens_q[b]:cu_seqlens_q[b+1]`` (int32
    ``[B+1]``); its query ``i`` is at position ``q_start[b] + i`` (int32 ``[B]``)
    and attends keys ``0..q_start[b]+i`` through ``block_tables[b]``. ``max_q_len``
    bounds the per-sequence query counts (host value, sizes the grid).
    ``plan``: the :func:`prefill_plan` of this metadata and shapes (heaviest
    work first, the heaviest items cut into merged key-range pieces).
    ``new_kv``: ``(k, v, slots)`` -- the step's new rows ``[N, H_kv, D]`` and
    their int64 write slots ``[N]`` -- written into the caches by the same
    launch (what :func:`kv_scatter` would do first); rows ``src_row0 ..
    src_row0 + total_q - 1`` are this call's query tokens, whose keys are then
    read from those rows (``ERR_WRITE_SLOT`` is flagged where a token's write
    slot is not its block-table slot).
    """
    dev = require_device(q, k_cache, v_cache, block_tables, cu_seqlens_q, q_start)
    _cache_layer("paged_prefill", k_cache)
    if q.dim() != 3:
        raise RuntimeError(f"paged_prefill: q must be [total_q, H_q, D], got {tuple(q.shape)}")
    total_q, hq, d = q.shape
    h_kv = k_cache.shape[1]
    if d != k_cache.shape[2] or q.dtype != k_cache.dtype or v_cache.shape != k_cache.shape:
        raise RuntimeError("paged_prefill: q / pool shape or dtype mismatch")
    if v_cache.stride() != k_cache.stride():
        raise RuntimeError("paged_prefill: k_cache and v_cache must share strides")
    b = block_tables.shape[0]
    if block_tables.dtype != torch.int32 or block_tables.dim() != 2 or block_tables.stride(1) != 1:
        raise RuntimeError("paged_prefill: block_tables must be int32 [B, max_blocks] with unit column stride")
    for name, t, n in (("cu_seqlens_q", cu_seqlens_q, b + 1), ("q_start", q_start, b)):
        if t.dtype != torch.int32 or t.shape != (n,) or not t.is_contiguous():
            raise RuntimeError(f"paged_prefill: {name} must be contiguous int32 [{n}]")
    _last_dim_contiguous("paged_prefill q", q)
    if plan is not None:
        require_device(q, plan.buf)
        if (plan.num_seqs, plan.max_q_len, plan.num_q_heads, plan.num_kv_heads, plan.head_dim) != (
                b, int(max_q_len), hq, h_kv, d):
            raise RuntimeError("paged_prefill: the plan was built for other shapes")
        if plan.f32 != (q.dtype == torch.float32):
            raise RuntimeError("paged_prefill: the plan was built for "
                               + ("fp32" if plan.f32 else "16-bit") + f" calls, q is {q.dtype}")
    if out is None:
        out = torch.empty(total_q, hq, d, dtype=q.dtype, device=dev)
    kn = vn = slots = None
    n_write = 0
    if new_kv is not None:
        kn, vn, slots = new_kv
        require_device(q, kn, vn, slots)
        n_write = kn.shape[0]
        if (kn.shape != (n_write, h_kv, d) or vn.shape != kn.shape or kn.dtype != q.dtype or vn.dtype != q.dtype
                or slots.dtype != torch.int64 or slots.shape != (n_write,)):
            raise RuntimeError("paged_prefill: new_kv must be (k, v [N, H_kv, D] of q's dtype, slots int64 [N])")
        _last_dim_contiguous("paged_prefill new k", kn)
        _last_dim_contiguous("paged_prefill new v", vn)
        slots = slots.contiguous()
    rc = lib().ir_paged_prefill(
        ptr(q), q.stride(0), q.stride(1), ptr(k_cache), ptr(v_cache), k_cache.stride(0), k_cache.stride(1),
        k_cache.shape[0] // block_size, block_size, ptr(block_tables), block_tables.stride(0),
        block_tables.shape[1], ptr(cu_seqlens_q), ptr(q_start), b, total_q, int(max_q_len), ptr(out),
        out.stride(0), out.stride(1), hq, h_kv, d, float(scale), dtype_code(q.dtype),
        None if plan is None else ptr(plan.buf), 0 if plan is None else plan.buf.numel(),
        ptr(kn), 0 if kn is None else kn.stride(0), 0 if kn is None else kn.stride(1),
        ptr(vn), 0 if vn is None else vn.stride(0), 0 if vn is None else vn.stride(1),
        ptr(slots), n_write, int(src_row0), ptr(err_flags), stream_ptr(dev),
    )
    check(rc, "ir_paged_prefill")
    return out


FORM_CLEAR_ON_FAIL = 1  # IR_FORM_CLEAR_ON_FAIL


def decode_form(gather_slots: torch.Tensor, mask: torch.Tensor, block_size: int, num_blocks: int,
                clear_on_fail: bool = False, host_verdict: torch.Tensor | None = None,
                tag: int = 0) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Block tables ``[B, ceil(T / bs)]`` int32 and context lengths ``[B]`` int32
    from the reference's decode metadata (``gather_slots`` ``[B, T]`` int64, mask
    ``[B, 1, 1, T]``), plus an int32 flag ``[1]``, nonzero unless the metadata
    has the reference engine's decode form exactly (``ir_decode_form``).
    ``clear_on_fail``: when the check fails, every context length is set to 0
    on the device (for a caller that does not wait for the flag).
    ``host_verdict``: a pinned int64 ``[1]`` host tensor the device writes
    ``tag << 32 | flag`` into at the end of the call."""
    dev = require_device(gather_slots, mask)
    if gather_slots.dtype != torch.int64 or gather_slots.dim() != 2:
        raise RuntimeError("decode_form: gather_slots must be int64 [B, T]")
    b, t = gather_slots.shape
    if mask.dim() != 4 or mask.shape[0] != b or mask.shape[1] != 1 or mask.shape[2] != 1 or mask.shape[3] != t:
        raise RuntimeError(f"decode_form: mask must be [B, 1, 1, T], got {tuple(mask.shape)}")
    if host_verdict is not None and (host_verdict.dtype != torch.int64 or host_verdict.numel() < 1
                                     or host_verdict.is_cuda):
        # (ir_decode_form refuses memory that is not pinned)
        raise RuntimeError("decode_form: host_verdict must be a pinned int64 host tensor")
    width = max(-(-t // block_size), 1)
    # one allocation: block tables | context lengths | flag and per-sequence flags
    n_bt = b * width
    buf = torch.empty(n_bt + 2 * b + 1, dtype=torch.int32, device=dev)
    base = buf.data_ptr()
    rc = lib().ir_decode_form(
        ptr(gather_slots), gather_slots.stride(0), gather_slots.stride(1), ptr(mask), mask.stride(0),
        mask.stride(3), dtype_code(mask.dtype), b, t, block_size, num_blocks, base, width, width,
        base + 4 * n_bt, base + 4 * (n_bt + b), FORM_CLEAR_ON_FAIL if clear_on_fail else 0, ptr(host_verdict),
        int(tag) & 0xFFFFFFFF, stream_ptr(dev),
    )
    check(rc, "ir_decode_form")
    return buf[:n_bt].view(b, width), buf[n_bt : n_bt + b], buf[n_bt + b : n_bt + b + 1]


@dataclass(slots=True)
class VarlenForm:
    """Prefill metadata derived from a reference packed frame: ``block_tables``
    ``[B, W]``, ``cu_seqlens_q`` ``[B + 1]`` and ``q_start`` ``[B]`` (int32,
    device) and the longest chunk ``max_q_len`` (host), with the step's prefill
    plan once built."""

    block_tables: torch.Tensor
    cu_seqlens_q: torch.Tensor
    q_start: torch.Tensor
    max_q_len: int
    q_lens: tuple[int, ...] = ()  # host copies of the derived chunk sizes and prefixes
    prefixes: tuple[int, ...] = ()
    prefill_plan: object | None = None
    row_split: object | None = None


def varlen_form(gather_slots: torch.Tensor, mask: torch.Tensor, block_size: int, num_blocks: int,
                records: torch.Tensor | None = None, staging: torch.Tensor | None = None,
                tables_capacity: int | None = None) -> VarlenForm | None:
    """Prefill metadata from the reference's packed prefill / mixed-step frame
    (``gather_slots`` ``[1, K]`` int64, mask ``[1, 1, Q, K]``), or ``None``
    unless it has that form exactly (``ir_varlen_form_scan``). Waits once:
    one call checks the mask and every slot on the device, derives the
    sequences, writes their block tables (stride read on the device) and
    publishes the verdict, the sizes, the chunk starts and the prefixes into
    ``staging``, tagged; the host polls the tag there (no stream
    synchronisation unless the wait runs long) and launches nothing more
    (``ir_varlen_form_tables`` only for tables beyond the call's table
    capacity).

    ``records``: int32 scratch of at least ``4 * Q`` elements, zero at rest
    (every call leaves it zero), 16-byte aligned; allocated zeroed when not
    given. ``staging``: a pinned host int32 tensor of at least
    :func:`varlen_staging_size` ``(Q)`` elements, written by the device (one
    caller at a time); without one the record is copied back from device
    memory after a stream synchronisation.
    ``tables_capacity``: block-table entries the call may write (default
    ``max(2**17, 4 * (K // block_size + Q))``); wider tables are written by a
    second launch after the read."""
    dev = require_device(gather_slots, mask)
    if gather_slots.dtype != torch.int64 or gather_slots.dim() != 2 or gather_slots.shape[0] != 1:
        raise RuntimeError("varlen_form: gather_slots must be int64 [1, K]")
    k = gather_slots.shape[1]
    if mask.dim() != 4 or tuple(mask.shape[:2]) != (1, 1) or mask.shape[3] != k:
        raise RuntimeError(f"varlen_form: mask must be [1, 1, Q, K], got {tuple(mask.shape)}")
    q = mask.shape[2]
    if q == 0 or k == 0 or q >= 2**31 or k >= 2**31:
        return None
    if records is None:
        records = torch.zeros(4 * q, dtype=torch.int32, device=dev)
    if records.dtype != torch.int32 or records.numel() < 4 * q or records.data_ptr() % 16:
        raise RuntimeError(f"varlen_form: records must be int32 [>= {4 * q}], 16-byte aligned, zero at rest")
    if staging is not None and (staging.dtype != torch.int32 or staging.is_cuda or not staging.is_contiguous()
                                or staging.numel() < 2 * q + 9):
        # (ir_varlen_form_scan refuses memory that is not pinned)
        raise RuntimeError(f"varlen_form: staging must be a pinned contiguous int32 host tensor of >= {2 * q + 9}")
    return varlen_form_checked(gather_slots, mask, block_size, num_blocks, records, staging,
                               None if staging is None else staging.numpy(), tables_capacity)


def varlen_form_checked(gather_slots: torch.Tensor, mask: torch.Tensor, block_size: int, num_blocks: int,
                        records: torch.Tensor, staging: torch.Tensor | None, host=None,
                        tables_capacity: int | None = None) -> VarlenForm | None:
    """:func:`varlen_form` once its checks have passed: the frame's shapes and
    dtypes (Q and K in [1, 2**31)), ``records`` and ``staging`` as that
    function requires them, and ``host`` a numpy view of ``staging`` (``None``
    without one). For a caller that holds its buffers across steps."""
    dev = mask.device
    q, k = mask.shape[2], mask.shape[3]
    # one allocation: info | cu | q_start | k_off | block tables (up to `cap`
    # entries); views are cut after the read, for what the form keeps
    o_cu, o_qs, o_ko, o_bt = _varlen_offsets(q)
    cap = max(1 << 17, 4 * (k // block_size + q)) if tables_capacity is None else max(int(tables_capacity), 0)
    cap = min(cap, 2**31 - 1)
    buf = torch.empty(o_bt + cap, dtype=torch.int32, device=dev)
    base = buf.data_ptr()
    pinned = staging is not None
    tag = (next(_record_tags) & 0x7FFFFFFF) or 1
    rc = lib().ir_varlen_form_scan(
        mask.data_ptr(), mask.stride(2), mask.stride(3), dtype_code(mask.dtype), q, k, gather_slots.data_ptr(),
        gather_slots.stride(1), block_size, num_blocks, records.data_ptr(), base + 4 * o_cu, base + 4 * o_qs,
        base + 4 * o_ko, base, base + 4 * o_bt, cap, staging.data_ptr() if pinned else None,
        staging.numel() if pinned else 0, tag, stream_ptr(dev),
    )
    check(rc, "ir_varlen_form_scan")
    if pinned:
        await_record(host, 7, tag, dev)
        bad, nseq, max_q, width, written = host[:5].tolist()
        if bad or nseq <= 0:
            return None
        rec = host[8 : 9 + 2 * nseq].tolist()
        offs, prefixes = rec[: nseq + 1], rec[nseq + 1 :]
    else:
        rec = buf[:o_ko].cpu()
        bad, nseq, max_q, width, written = rec[:5].tolist()
        if bad or nseq <= 0:
            return None
        offs, prefixes = rec[o_cu : o_cu + nseq + 1].tolist(), rec[o_qs : o_qs + nseq].tolist()
    width = max(width, 1)
    cu = buf.as_strided((nseq + 1,), (1,), o_cu)
    q_start = buf.as_strided((nseq,), (1,), o_qs)
    if written:
        bt = buf.as_strided((nseq, width), (width, 1), o_bt)
    else:
        bt = torch.empty(nseq, width, dtype=torch.int32, device=dev)
        rc = lib().ir_varlen_form_tables(
            gather_slots.data_ptr(), gather_slots.stride(1), base + 4 * o_ko, cu.data_ptr(), q_start.data_ptr(),
            nseq, block_size, bt.data_ptr(), bt.stride(0), width, stream_ptr(dev),
        )
        check(rc, "ir_varlen_form_tables")
    q_lens = tuple(b - a_ for a_, b in zip(offs, offs[1:]))
    return VarlenForm(bt, cu, q_start, max_q, q_lens, tuple(prefixes))


_record_tags = itertools.count(1)  # tags of the device-written host records, never reused in a process
RECORD_POLLS = 30_000  # polls of a host record (~2 ms) before a stream synchronisation instead


def await_record(host, word: int, tag: int, dev: torch.device) -> None:
    """Waits until ``host[word]`` (a numpy view of pinned memory the device
    writes, the tag word last) holds ``tag``: polls it up to ``RECORD_POLLS``
    times, which sees the record as soon as the device has written it, then
    synchronises the stream; raises if the record is still not there."""
    for _ in range(RECORD_POLLS):
        if host[word] == tag:
            return
    torch.cuda.current_stream(dev).synchronize()
    if host[word] != tag:
        raise RuntimeError("the device wrote no record for this call")


def _varlen_offsets(q: int) -> tuple[int, int, int, int]:
    """Element offsets of cu_seqlens_q, q_start, the key offsets and the block
    tables in the check's buffer (info at 0; 256-byte regions)."""
    a = (q + 1 + 63) // 64 * 64
    b = (q + 63) // 64 * 64
    return 64, 64 + a, 64 + a + b, 64 + a + 2 * b


def varlen_staging_size(q: int) -> int:
    """int32 elements of the pinned host record :func:`varlen_form` has the
    device write (the verdict and sizes, then up to ``q + 1`` chunk starts and
    ``q`` prefixes)."""
    return (2 * q + 9 + 63) // 64 * 64


def stream_capture_id(device: torch.device | str | int | None = None) -> int:
    """0 unless torch's current stream on ``device`` is capturing a graph; then
    a value unique to that capture (``ir_stream_capture_id``)."""
    import ctypes

    dev = torch.device(device if device is not None else "cuda")
    out = ctypes.c_uint64(0)
    check(lib().ir_stream_capture_id(stream_ptr(dev), ctypes.byref(out)), "ir_stream_capture_id")
    return int(out.value)


def hbm_read(src: torch.Tensor, sink: torch.Tensor, workgroups: int = 0) -> None:
    """Reads all of ``src`` (contiguous, a multiple of :func:`hbm_read_granule`
    bytes) with the decode kernels' load form and discards it: timing it gives
    the device's read-only HBM roof. ``sink``: an int32 tensor of >= 1 element."""
    dev = require_device(src, sink)
    nbytes = src.numel() * src.element_size()
    if not src.is_contiguous() or nbytes % hbm_read_granule():
        raise RuntimeError(f"hbm_read: src must be contiguous and a multiple of {hbm_read_granule()} bytes")
    if sink.dtype != torch.int32 or sink.numel() < 1:
        raise RuntimeError("hbm_read: sink must be an int32 tensor")
    check(lib().ir_hbm_read(ptr(src), nbytes, ptr(sink), int(workgroups), stream_ptr(dev)), "ir_hbm_read")


def hbm_read_granule() -> int:
    return int(lib().ir_hbm_read_granule())


__all__ = [
    "kv_scatter",
    "gather_slots",
    "paged_gather",
    "paged_decode",
    "paged_attention_masked",
    "paged_prefill",
    "PrefillPlan",
    "prefill_plan",
    "prefill_plan_bytes",
    "prefill_plan_pays",
    "rope_kv_scatter",
    "decode_workspace_bytes",
    "default_partition",
]
