"""Shared paged K/V pool and per-forward paged metadata (MI355X build).

Same public surface as the reference's ``infrared/cache/paged_kv_cache.py``:

- ``PagedKVPool(num_layers, num_blocks, block_size, num_kv_heads, head_dim,
  dtype, device)`` with ``.k`` / ``.v`` of shape ``[num_layers, num_blocks *
  block_size, num_kv_heads, head_dim]`` (``infrared/cache/paged_kv_cache.py:30-46``),
  ``.write(layer_idx, k, v, slots)`` (``:48-57``) and ``.gather(layer_idx,
  gather_slots)`` (``:59-72``).
- ``PagedContext(pool, write_slots, gather_slots, use_triton=True)``
  (``:75-91``), with optional device-side fields the fast kernels read:
  ``block_tables`` ``[B, max_blocks]`` int32, ``context_lens`` ``[B]`` int32.

Indexing is the reference's: ``pool.k[layer, s]`` is the ``[num_kv_heads,
head_dim]`` row of slot ``s`` and callers may write ``pool.k[layer, a:b]``
directly. The physical layout is a choice:

- ``layout="head_major"`` (default): storage ``[L, num_kv_heads, num_slots,
  head_dim]``, exposed as the ``[L, num_slots, num_kv_heads, head_dim]`` view.
  One KV head's block of 16 tokens is then 16 * head_dim contiguous elements
  (4 KiB in bf16 at head_dim 128), which the decode kernel streams with
  fully contiguous 1 KiB load instructions.
- ``layout="slot_major"``: the reference's contiguous ``[L, num_slots,
  num_kv_heads, head_dim]`` storage (a KV head's block is 16 pieces of
  ``head_dim`` elements strided by a whole slot row).

Every kernel takes the slot and head strides, so both layouts run the same
code. ``write`` runs the HIP scatter kernel; ``gather`` runs the HIP
slot-gather. The pool lives in device memory only: CPU tensors are rejected
rather than handled by a fallback.
"""

from __future__ import annotations

import weakref
from collections.abc import Sequence
from dataclasses import dataclass, field

import numpy as np
import torch

from infrared_amd import kernels
from infrared_amd._lib import (
    ERR_BLOCK_RANGE,
    ERR_CONTEXT_RANGE,
    ERR_GATHER_RANGE,
    ERR_PLAN,
    ERR_SLOT_RANGE,
    ERR_WRITE_SLOT,
)

_ERR_NAMES = {
    ERR_SLOT_RANGE: "write slot outside the pool",
    ERR_BLOCK_RANGE: "block id outside the pool",
    ERR_CONTEXT_RANGE: "context length outside the block table",
    ERR_GATHER_RANGE: "gather slot outside the pool",
    ERR_PLAN: "decode plan with sequence pairs run without share groups",
    ERR_WRITE_SLOT: "new token written elsewhere than its block-table slot",
}


class PagedKVPool:
    """Flat K/V slot pool on a ROCm device, addressed by slot id ``block * size + off``.

    ``strict=True`` synchronises after every kernel and raises on any
    out-of-range slot / block id the kernels flagged (debug mode). Otherwise
    flags accumulate on the device and ``check_errors()`` reports them.
    """

    def __init__(
        self,
        num_layers: int,
        num_blocks: int,
        block_size: int,
        num_kv_heads: int,
        head_dim: int,
        dtype: torch.dtype,
        device: torch.device | str = "cuda",
        *,
        strict: bool = False,
        layout: str = "head_major",
    ) -> None:
        device = torch.device(device)
        if device.type != "cuda":
            raise RuntimeError(
                f"PagedKVPool lives in ROCm device memory; device {device} is not supported"
            )
        self.num_layers = num_layers
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.num_slots = num_blocks * block_size
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.device = device
        self.strict = strict
        self.layout = layout
        if layout == "head_major":
            store = (num_layers, num_kv_heads, self.num_slots, head_dim)
            self.k = torch.zeros(store, dtype=dtype, device=device).permute(0, 2, 1, 3)
            self.v = torch.zeros(store, dtype=dtype, device=device).permute(0, 2, 1, 3)
        elif layout == "slot_major":
            shape = (num_layers, self.num_slots, num_kv_heads, head_dim)
            self.k = torch.zeros(shape, dtype=dtype, device=device)
            self.v = torch.zeros(shape, dtype=dtype, device=device)
        else:
            raise ValueError(f"unknown pool layout {layout!r} (head_major, slot_major)")
        self.err_flags = torch.zeros(1, dtype=torch.int32, device=device)
        self._workspace: torch.Tensor | None = None
        self._counters: torch.Tensor | None = None
        self._plan_buf: torch.Tensor | None = None
        # the decode plan whose schedule plan_buffer() holds now: a context
        # whose cached plan is not this one was overwritten and rebuilds it
        self.plan_owner: object | None = None
        # (metadata key, derived form) of the last eager reference-form check
        self._ref_form: tuple | None = None
        self._ref_varlen: tuple | None = None
        # decode forms recorded into a graph under capture, by (capture id,
        # id(gather_slots), id(mask)): each holds the buffers its graph's
        # replays address and lives as long as the captured gather_slots
        self._captured_forms: dict[tuple, tuple] = {}
        # the packed-form check's row records (zero at rest), pinned record and its numpy view
        self._varlen_records: torch.Tensor | None = None
        self._varlen_staging: torch.Tensor | None = None
        self._varlen_host = None
        # the eager decode-form check's verdict, written by the device into
        # pinned memory as tag << 32 | flag (read without synchronising)
        self._verdict: torch.Tensor | None = None
        self._verdict_np = None
        self._verdict_tag = 0

    # --- reference surface ------------------------------------------------

    def write(
        self, layer_idx: int, k: torch.Tensor, v: torch.Tensor, slots: torch.Tensor
    ) -> None:
        """Scatter this step's K/V (``[N, num_kv_heads, head_dim]``) into ``slots`` (``[N]`` int64)."""
        kernels.kv_scatter(self.k[layer_idx], self.v[layer_idx], k, v, slots, self.err_flags)
        if self.strict:
            self.check_errors()

    def gather(
        self, layer_idx: int, gather_slots: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """Per-query histories: ``gather_slots`` ``[B, T]`` int64 -> ``[B, T, H, D]`` K and V.

        Same values as the reference's ``self.k[layer_idx, flat]`` indexing, read
        by the HIP slot-gather kernel. A slot outside the pool reads as zeros and
        is flagged (``IndexError`` from ``check_errors()``, or at once when strict).
        """
        out = kernels.gather_slots(self.k[layer_idx], self.v[layer_idx], gather_slots, self.err_flags)
        if self.strict:
            self.check_errors()
        return out

    # --- MI355X additions ---------------------------------------------------

    def gather_blocks(
        self,
        layer_idx: int,
        block_tables: torch.Tensor,
        context_lens: torch.Tensor,
        max_ctx: int,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """Dense zero-padded histories ``[B, max_ctx, H, D]`` through block tables (HIP kernel)."""
        out = kernels.paged_gather(
            self.k[layer_idx], self.v[layer_idx], block_tables, context_lens,
            self.block_size, max_ctx, self.err_flags,
        )
        if self.strict:
            self.check_errors()
        return out

    def workspace(self, nbytes: int) -> torch.Tensor:
        """A cached device buffer of at least ``nbytes`` for the decode kernels'
        fp32 partial rows (scratch, any shape).

        Grow it outside hipGraph capture (the graph decoder's warm-up does).
        Growing replaces the tensor: a graph captured on the old one must hold a
        reference to it (the graph decoder does) to keep its memory alive.
        """
        if self._workspace is None or self._workspace.numel() < nbytes:
            self._workspace = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=self.device)
        return self._workspace

    def decode_counters(self, n: int) -> torch.Tensor:
        """A cached int32 buffer of at least ``n`` arrival counters, zero at rest:
        every decode call leaves the counters it used at zero, so calls of any
        batch shape share it. Grown (zero-filled) outside hipGraph capture."""
        if self._counters is None or self._counters.numel() < n:
            self._counters = torch.zeros(max(n, 64), dtype=torch.int32, device=self.device)
        return self._counters

    def plan_buffer(self, nbytes: int) -> torch.Tensor:
        """A cached device buffer of at least ``nbytes`` for the decode plan of
        the current step (rebuilt by each step's first decode layer; steps are
        stream-ordered). Grown outside hipGraph capture, like the workspace."""
        if self._plan_buf is None or self._plan_buf.numel() < nbytes:
            self._plan_buf = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=self.device)
        return self._plan_buf

    def reference_decode_form(self, gather_slots: torch.Tensor, mask: torch.Tensor) -> _DecodeForm | None:
        """Block tables for the reference engine's decode metadata, if it has the
        decode form; else ``None`` (the caller runs the mask kernel).

        The reference's eager decode builds ``gather_slots[i, p] = bt_i[p // bs]
        * bs + p % bs`` for ``p < ctx_i`` (0 after) and an additive mask of 0 for
        ``p < ctx_i`` and ``finfo(dtype).min`` after
        (``infrared/engine/paged_engine.py:306-314, 630-638``). Derived on the
        device by ``ir_decode_form`` -- ``bt_i[j] = gather_slots[i, j * bs] //
        bs``, ``ctx_i`` = the mask's zeros -- and verified exactly: every slot
        below ``ctx_i`` follows the closed form, the zeros are a nonempty
        prefix, and every later mask value is at most -6e4 (masked in any
        dtype, fp16's ``finfo.min`` included), so the decode kernels compute
        what the mask kernel would.

        The host never waits for the check. It runs with
        ``IR_FORM_CLEAR_ON_FAIL`` and the returned form carries its device flag
        as ``gate``: until the verdict is known the caller runs the block-table
        decode followed by the mask kernel gated on the flag (each replay, or
        each call, then computes what the mask kernel would). Eagerly the
        device also writes the verdict, tagged, into the pool's pinned record;
        :meth:`_DecodeForm.verdict` reads it there when it has arrived (by the
        step's second layer, typically), and later layers then run only the
        kernels it selects. The eager result is cached for the step's other
        layers (same ``gather_slots`` and ``mask`` tensors, not modified in
        place since).

        Under hipGraph capture (the reference's ``CudaGraphDecoder`` captures
        its decode forward on static ``gather_slots`` / ``mask`` buffers that
        each replay refills, ``infrared/engine/cuda_graph.py:231-285``) the
        check itself is recorded, once per capture and metadata pair, and its
        form never reads a verdict: each replay checks its own metadata and
        runs the block-table kernels in the decode form, otherwise the mask
        kernel. The eager cache is never consulted under capture. The form
        holds the buffers its graph addresses (its own plan buffer, the decode
        workspace and counters) for as long as the captured ``gather_slots``
        tensor lives.
        """
        if not (gather_slots.dim() == 2 and gather_slots.dtype == torch.int64 and gather_slots.is_cuda
                and mask.is_cuda and mask.dim() == 4 and tuple(mask.shape[:3]) == (gather_slots.shape[0], 1, 1)
                and mask.shape[3] == gather_slots.shape[1]):
            return None
        if torch.cuda.is_current_stream_capturing():
            return self._captured_decode_form(gather_slots, mask)
        c = self._ref_form
        if c is not None and _same_metadata(c[0], gather_slots, mask):
            return c[1]
        if self._verdict is None:
            self._verdict = torch.zeros(1, dtype=torch.int64, pin_memory=True)
            self._verdict_np = self._verdict.numpy()  # the same pinned memory, read without torch
        self._verdict_tag = (self._verdict_tag + 1) & 0x7FFFFFFF
        bt, ctx, bad = kernels.decode_form(gather_slots, mask, self.block_size, self.num_blocks,
                                           clear_on_fail=True, host_verdict=self._verdict, tag=self._verdict_tag)
        form = _DecodeForm(bt, ctx, gate=bad, peek=(self._verdict_np, self._verdict_tag))
        self._ref_form = (_metadata_key(gather_slots, mask), form)
        return form

    def _captured_decode_form(self, gather_slots: torch.Tensor, mask: torch.Tensor) -> _DecodeForm:
        cid = kernels.stream_capture_id(gather_slots.device)
        slot = (cid, id(gather_slots), id(mask))
        c = self._captured_forms.get(slot)
        if c is not None and _same_metadata(c[0], gather_slots, mask):
            return c[1]
        bt, ctx, bad = kernels.decode_form(gather_slots, mask, self.block_size, self.num_blocks,
                                           clear_on_fail=True)
        form = _DecodeForm(bt, ctx, gate=bad)
        self._captured_forms[slot] = (_metadata_key(gather_slots, mask), form)
        weakref.finalize(gather_slots, _drop_captured, weakref.ref(self), slot)
        return form

    def reference_varlen_form(self, gather_slots: torch.Tensor, mask: torch.Tensor) -> kernels.VarlenForm | None:
        """Chunked-prefill metadata for the reference engine's packed prefill
        frame, if it has that form; else ``None`` (the caller runs the mask
        kernel).

        The reference's prefix-hit prefill and mixed steps pass one frame (batch
        1) of Q query tokens, a key axis concatenating each scheduled sequence's
        history ``[0, start + q)`` in order, ``gather_slots[1, K]`` with the
        closed form per sequence and the additive mask of
        ``build_attention_mask`` / ``build_varlen_mask``
        (``infrared/engine/paged_engine.py:194-206, 461-516``,
        ``infrared/model/inputs.py:33-85``). ``ir_varlen_form_scan`` recovers
        ``cu_seqlens_q``, ``q_start`` and the block tables on the device and
        verifies the form exactly, so the chunked-prefill kernel computes what
        the mask kernel would. The check reads the mask once and the host
        waits once, polling the pool's pinned record, which the device writes
        (verdict, sizes, chunk starts and prefixes, then a tag) at the end of
        the call; the result is cached for the step's other layers (same
        ``gather_slots`` and ``mask`` tensors, not modified in place since).
        Under hipGraph capture ``None`` is returned and the mask kernel runs.
        """
        if torch.cuda.is_current_stream_capturing():
            return None
        c = self._ref_varlen
        if c is not None and _same_metadata(c[0], gather_slots, mask):
            return c[1]
        form = None
        if (gather_slots.dim() == 2 and gather_slots.shape[0] == 1 and gather_slots.dtype == torch.int64
                and gather_slots.is_cuda and mask.device == gather_slots.device and mask.dim() == 4
                and tuple(mask.shape[:2]) == (1, 1) and mask.shape[3] == gather_slots.shape[1]
                and 0 < mask.shape[2] < 2**31 and 0 < mask.shape[3] < 2**31):
            q = mask.shape[2]
            if self._varlen_records is None or self._varlen_records.numel() < 4 * q:
                self._varlen_records = torch.zeros(max(4 * q, 1024), dtype=torch.int32, device=self.device)
                self._varlen_staging = torch.zeros(kernels.varlen_staging_size(max(q, 256)), dtype=torch.int32,
                                                   pin_memory=True)
                self._varlen_host = self._varlen_staging.numpy()  # the same pinned memory
            form = kernels.varlen_form_checked(gather_slots, mask, self.block_size, self.num_blocks,
                                               self._varlen_records, self._varlen_staging, self._varlen_host)
            if form is not None:
                # the reference packs decodes first (infrared/engine/scheduler.py:104-115)
                form.row_split = row_split(form.block_tables, form.prefixes, form.q_lens)
        self._ref_varlen = (_metadata_key(gather_slots, mask), form)
        return form

    def check_errors(self) -> None:
        """Synchronises, raises ``IndexError`` for any flagged range error, then clears the flags."""
        flags = int(self.err_flags.item())
        if flags:
            self.err_flags.zero_()
            names = [n for bit, n in _ERR_NAMES.items() if flags & bit]
            raise IndexError("paged kernels flagged: " + ", ".join(names))


def _metadata_key(gather_slots: torch.Tensor, mask: torch.Tensor) -> tuple:
    """Identity of a step's metadata for the form caches: weak references to
    the two tensors (a cache entry pins neither, and a dead reference matches
    nothing, so a reused id is never mistaken for them) and their in-place
    version counters, so a caller that refills the same tensors for the next
    step is checked again."""
    return (weakref.ref(gather_slots), gather_slots._version, weakref.ref(mask), mask._version)


def _same_metadata(key: tuple, gather_slots: torch.Tensor, mask: torch.Tensor) -> bool:
    return (key[0]() is gather_slots and key[1] == gather_slots._version and key[2]() is mask
            and key[3] == mask._version)


def _drop_captured(pool_ref, slot) -> None:
    pool = pool_ref()
    if pool is not None:
        pool._captured_forms.pop(slot, None)


@dataclass(slots=True)
class _DecodeForm:
    """Block tables and context lengths derived from reference decode metadata,
    with the step's decode plan once built.

    ``gate`` is the check's int32 flag on the device, nonzero when the
    metadata is not in the decode form (the context lengths are then 0); a
    form with a gate has its own ``plan_buf``. ``peek`` (eager forms): the
    pinned record the device writes the tagged verdict into, and the tag;
    ``held`` keeps the pool buffers a captured graph's kernels address alive."""

    block_tables: torch.Tensor
    context_lens: torch.Tensor
    decode_plan: object | None = None
    gate: torch.Tensor | None = None
    plan_buf: torch.Tensor | None = None
    held: list = field(default_factory=list)
    peek: tuple | None = None

    def verdict(self) -> bool | None:
        """True / False once the device has published this form's check (the
        metadata is / is not in the decode form), None before (or for a form
        recorded under capture, which never reads one)."""
        if self.peek is None:
            return None
        record, tag = self.peek
        v = int(record[0])
        if v >> 32 != tag:
            return None
        return (v & 0xFFFFFFFF) == 0


@dataclass(slots=True)
class RowSplit:
    """A packed step divided by kernel: its one-token rows (decodes), one block
    of packed rows ``dec_range`` = (first, end), run as a decode batch
    (``dec_tables``, ``dec_ctx`` = contexts including the new token, int32);
    the other sequences' rows, the block ``pre_range``, as chunked prefill
    (``pre_tables``, ``pre_cu``, ``pre_q_start``, ``pre_max_q``). The parts'
    plans are cached here for the step's other layers."""

    dec_range: tuple[int, int]
    dec_tables: torch.Tensor
    dec_ctx: torch.Tensor
    pre_range: tuple[int, int]
    pre_tables: torch.Tensor
    pre_cu: torch.Tensor
    pre_q_start: torch.Tensor
    pre_max_q: int
    decode_plan: object | None = None
    prefill_plan: object | None = None


def row_split(bt: torch.Tensor, num_cached: Sequence[int], q_lens: Sequence[int]) -> RowSplit | None:
    """The packed step's one-token rows as a decode batch and the rest as
    chunked prefill, when those rows form one block (the decodes packed first
    or last, as a scheduler lists them); else ``None`` (one prefill launch, no
    row copies)."""
    dec = [i for i, n in enumerate(q_lens) if n == 1]
    if not dec or dec != list(range(dec[0], dec[0] + len(dec))):
        return None
    if dec[0] != 0 and dec[-1] != len(q_lens) - 1:
        return None
    pre = [i for i, n in enumerate(q_lens) if n > 1]
    first = sum(q_lens[: dec[0]])  # packed row of the first decode
    nd = len(dec)
    dec_range = (first, first + nd)
    total = sum(q_lens)
    pre_range = (nd, total) if first == 0 else (0, first)
    pre_cu = np.concatenate([[0], np.cumsum([q_lens[i] for i in pre], dtype=np.int64)])
    host = torch.from_numpy(np.concatenate([
        np.asarray(dec, np.int64), np.asarray(pre, np.int64), np.asarray([num_cached[i] + 1 for i in dec], np.int64),
        pre_cu, np.asarray([num_cached[i] for i in pre], np.int64)]).astype(np.int64))
    t = host.to(bt.device)  # one host->device copy
    dec_idx, pre_idx, dec_ctx, pre_cu_t, pre_qs = torch.split(t, [nd, len(pre), nd, len(pre) + 1, len(pre)])
    return RowSplit(
        dec_range=dec_range,
        dec_tables=bt.index_select(0, dec_idx).contiguous(),
        dec_ctx=dec_ctx.to(torch.int32),
        pre_range=pre_range,
        pre_tables=bt.index_select(0, pre_idx).contiguous(),
        pre_cu=pre_cu_t.to(torch.int32),
        pre_q_start=pre_qs.to(torch.int32),
        pre_max_q=max((q_lens[i] for i in pre), default=0),
    )


@dataclass(slots=True)
class PagedContext:
    """Per-forward paged metadata handed to the attention layer.

    ``write_slots`` ``[N]`` int64 — flat slots of this step's new K/V, in query
    token order. ``gather_slots`` ``[B, T]`` int64 — per query row, the slots of
    its history (right-padded), read together with the caller's additive mask.
    ``use_triton`` keeps the reference's field name: ``True`` lets the dispatcher
    take the block-table kernels when their fields are present; ``False``
    forces the kernel that reads ``gather_slots`` + mask. All are HIP kernels;
    there is no Triton and no CPU path.

    Block-table fields (additions; the reference's context has none):
    ``block_tables`` ``[B, max_blocks]`` int32 per sequence; for a one-token
    decode ``context_lens`` ``[B]`` int32; for prefill / mixed steps over
    packed query tokens ``cu_seqlens_q`` ``[B + 1]`` int32 (sequence ``b`` owns
    packed rows ``cu[b]:cu[b+1]``), ``q_start`` ``[B]`` int32 (its cached
    prefix length) and ``max_q_len`` (host bound on the chunk sizes).
    ``decode_plan`` caches the balanced decode schedule of ``block_tables`` /
    ``context_lens``, ``prefill_plan`` the heaviest-first work plan of a
    prefill step: the step's first layer builds them, the others reuse them (a
    context is one step's metadata, shared by every layer). ``row_split``
    (from ``metadata.prefill_context``, for a packed step whose one-token rows
    form one block) sends those rows to the decode kernels and the chunks to
    the prefill kernel.
    """

    pool: PagedKVPool
    write_slots: torch.Tensor
    gather_slots: torch.Tensor | None = None
    use_triton: bool = True
    block_tables: torch.Tensor | None = None
    context_lens: torch.Tensor | None = None
    cu_seqlens_q: torch.Tensor | None = None
    q_start: torch.Tensor | None = None
    max_q_len: int = 0
    decode_plan: object | None = None
    prefill_plan: object | None = None
    row_split: RowSplit | None = None
