"""The attention seam: ``paged_attention(q, k, v, paged, mask, layer_idx, scale, n_rep)``.

Same signature and contract as the reference dispatcher
(``infrared/model/triton_attention.py:81-107``), which ``Attention.forward``
calls once per layer (``infrared/model/layers.py:178-180``):

1. scatter this step's K/V into the pool at ``paged.write_slots`` (HIP scatter
   kernel, ``infrared/model/triton_attention.py:101-104``);
2. attend over the paged history with a HIP kernel:

   - ``paged.use_triton``, 16-bit dtype and ``paged.block_tables`` +
     ``paged.cu_seqlens_q`` + ``paged.q_start`` set: the chunked-prefill MFMA
     kernel over the packed query tokens (prefix-hit prefill and mixed
     prefill + decode steps); the mask is implied: query ``i`` of sequence
     ``b`` sees keys ``<= q_start[b] + i`` of its own sequence (the masks of
     ``infrared/model/inputs.py:33-85``);
   - ``paged.use_triton`` and ``paged.block_tables``/``paged.context_lens`` set
     and one query token per sequence: the GQA decode kernel (split-KV +
     log-sum-exp reduce) over the block tables; the mask is then implied by
     ``context_lens`` (key ``t`` valid iff ``t < context_lens[b]``, the decode
     mask of ``infrared/engine/paged_engine.py:630-638``);
   - otherwise, for a one-token decode whose ``gather_slots`` + ``mask`` have
     the reference engine's decode form (``gather_slots[i, p] = bt[p // bs] *
     bs + p % bs`` and mask 0 then ``finfo.min``,
     ``infrared/engine/paged_engine.py:306-314, 630-638``): the same decode
     kernels over block tables derived from them on the device (checked once
     per step, ``PagedKVPool.reference_decode_form``, with no host wait: until
     the check's verdict reaches the host -- under graph capture, never -- its
     flag gates, on the device, a mask kernel run after the decode, so each
     call or replay takes the path its own metadata allows);
   - otherwise, for the reference engine's packed prefill / mixed-step frame
     (batch 1: every scheduled sequence's query tokens, a key axis
     concatenating their histories in order, ``gather_slots`` with the closed
     form per sequence and the mask of ``build_attention_mask`` /
     ``build_varlen_mask``, ``infrared/engine/paged_engine.py:194-206,
     461-516``): the chunked-prefill kernel over ``cu_seqlens_q``, ``q_start``
     and block tables derived from them on the device (checked once per step,
     ``PagedKVPool.reference_varlen_form``);
   - otherwise: the kernel that reads ``gather_slots`` + the additive ``mask``
     exactly as the reference's naive path does
     (``infrared/model/triton_attention.py:110-129``).

``paged`` may be this package's ``PagedContext`` or any object with the same
attributes (the reference's own ``PagedContext`` works: it simply lacks the
block-table fields). There is no CPU path and no Triton: tensors must live on
the ROCm device and the HIP library must be built.
"""

from __future__ import annotations

import torch

from infrared_amd import kernels


def paged_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    paged,
    mask: torch.Tensor | None,
    layer_idx: int,
    scale: float,
    n_rep: int,
) -> torch.Tensor:
    """Write this step's K/V into the pool, then attend over the paged history.

    ``q`` ``[B, Sq, H, D]`` (RoPE applied); ``k``/``v`` ``[B, Sq, H_kv, D]``;
    ``mask`` ``[B, 1, Sq, T]`` additive (may be ``None`` on the block-table path).
    Returns ``[B, Sq, H, D]``. Where the call runs the chunked-prefill kernel
    the write is part of that launch (``ir_paged_prefill``'s fused write: the
    kernel reads its own new keys from ``k`` / ``v``); elsewhere
    ``pool.write`` runs first.
    """
    h_kv, d = k.shape[-2], k.shape[-1]
    b, sq, hq, dq = q.shape
    if dq != d or hq != h_kv * n_rep:
        raise RuntimeError(
            f"paged_attention: q {tuple(q.shape)} inconsistent with k {tuple(k.shape)} and n_rep={n_rep}"
        )
    return _attend(q, paged, mask, layer_idx, scale,
                   new_kv=(k.reshape(-1, h_kv, d), v.reshape(-1, h_kv, d), paged.write_slots))


def rope_paged_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    paged,
    mask: torch.Tensor | None,
    layer_idx: int,
    scale: float,
    n_rep: int,
) -> torch.Tensor:
    """``apply_rotary_pos_emb`` + ``paged_attention`` with the rotation and the K/V
    write fused into one kernel (``ir_rope_kv_scatter``).

    Takes the pre-RoPE ``q``/``k`` of ``Attention.forward``
    (``infrared/model/layers.py:158-164``) and the step's fp32 ``cos``/``sin``
    ``[B, Sq, D]`` (``RotaryEmbedding`` output); the result is bit-identical to
    rotating with the reference's ops and calling ``paged_attention``.
    """
    pool = paged.pool
    h_kv, d = k.shape[-2], k.shape[-1]
    b, sq, hq, dq = q.shape
    if dq != d or hq != h_kv * n_rep:
        raise RuntimeError(
            f"rope_paged_attention: q {tuple(q.shape)} inconsistent with k {tuple(k.shape)} and n_rep={n_rep}"
        )
    q_rot = kernels.rope_kv_scatter(
        q.reshape(b * sq, hq, d), k.reshape(b * sq, h_kv, d), v.reshape(b * sq, h_kv, d),
        cos.reshape(b * sq, d), sin.reshape(b * sq, d), pool.k[layer_idx], pool.v[layer_idx],
        paged.write_slots, err_flags=getattr(pool, "err_flags", None),
    ).view(b, sq, hq, d)
    return _attend(q_rot, paged, mask, layer_idx, scale)


def _attend(q: torch.Tensor, paged, mask: torch.Tensor | None, layer_idx: int, scale: float,
            new_kv: tuple | None = None) -> torch.Tensor:
    """Attention over the pool. ``new_kv`` = (k rows, v rows, write slots) of
    this step, not yet written: the chunked-prefill paths fold the write into
    their launch, every other path writes them first (``pool.write``)."""
    pool = paged.pool
    b, sq = q.shape[:2]
    k_layer, v_layer = pool.k[layer_idx], pool.v[layer_idx]
    err = getattr(pool, "err_flags", None)
    fusable = new_kv is not None and _fusable(pool, layer_idx, new_kv)

    def write():
        if new_kv is not None:
            pool.write(layer_idx, *new_kv)

    block_tables = getattr(paged, "block_tables", None)
    context_lens = getattr(paged, "context_lens", None)
    cu_seqlens_q = getattr(paged, "cu_seqlens_q", None)
    q_start = getattr(paged, "q_start", None)
    if (
        paged.use_triton
        and block_tables is not None
        and cu_seqlens_q is not None
        and q_start is not None
        and q.dtype in (torch.bfloat16, torch.float16, torch.float32)
    ):
        split = getattr(paged, "row_split", None)
        if not fusable:
            write()
        if split is not None:
            out = _split_step(q, pool, layer_idx, split, scale, err, new_kv if fusable else None)
        else:
            max_q = getattr(paged, "max_q_len", 0) or b * sq
            out = _prefill(q, pool, layer_idx, block_tables, cu_seqlens_q, q_start, max_q, paged, scale, err,
                           new_kv=new_kv if fusable else None)
    elif paged.use_triton and block_tables is not None and context_lens is not None and sq == 1:
        write()
        out = _decode(q, pool, layer_idx, block_tables, context_lens, paged, scale, err)
    else:
        if paged.gather_slots is None or mask is None:
            raise RuntimeError(
                "paged_attention: gather_slots and mask are required unless block_tables/"
                "context_lens drive a single-token decode"
            )
        form = None
        if (paged.use_triton and sq == 1 and hasattr(pool, "reference_decode_form")
                and paged.gather_slots.dim() == 2 and paged.gather_slots.shape[0] == b):
            # the reference's own decode metadata (gather_slots + mask, no block
            # tables): when it has the decode form, run the block-table kernels
            form = pool.reference_decode_form(paged.gather_slots, mask)
        vform = None
        if (form is None and paged.use_triton and b == 1
                and q.dtype in (torch.bfloat16, torch.float16, torch.float32)
                and hasattr(pool, "reference_varlen_form") and mask.dim() == 4 and mask.shape[2] == sq):
            # the reference's packed prefill / mixed-step frame: when it has
            # that form, run the chunked-prefill kernel over derived metadata
            vform = pool.reference_varlen_form(paged.gather_slots, mask)
        if vform is None or not fusable:
            write()
            fusable = False
        verdict = form.verdict() if form is not None else None
        if form is not None and verdict is False:
            # the check's published verdict: not the decode form
            out = kernels.paged_attention_masked(
                q, k_layer, v_layer, paged.gather_slots, mask, scale, err_flags=err
            )
        elif form is not None:
            out = _decode(q, pool, layer_idx, form.block_tables, form.context_lens, form, scale, err)
            verdict = form.verdict()  # (it may have arrived while the decode was launched)
            if form.gate is not None and verdict is not True:
                # verdict not known on the host (under capture, never): the
                # check's flag decides, on the device, whether this mask kernel
                # overwrites the rows; known to fail: it does
                kernels.paged_attention_masked(
                    q, k_layer, v_layer, paged.gather_slots, mask, scale, out=out, err_flags=err,
                    run_if=form.gate if verdict is None else None,
                )
        elif vform is not None and vform.row_split is not None:
            out = _split_step(q, pool, layer_idx, vform.row_split, scale, err, new_kv if fusable else None)
        elif vform is not None:
            out = _prefill(q, pool, layer_idx, vform.block_tables, vform.cu_seqlens_q, vform.q_start,
                           vform.max_q_len, vform, scale, err, new_kv=new_kv if fusable else None)
        else:
            out = kernels.paged_attention_masked(
                q, k_layer, v_layer, paged.gather_slots, mask, scale, err_flags=err
            )
    if getattr(pool, "strict", False):
        pool.check_errors()
    return out


def _split_step(q, pool, layer_idx: int, split, scale: float, err, new_kv: tuple | None = None) -> torch.Tensor:
    """A packed step whose one-token rows (decodes) form one block of rows:
    those rows through the decode kernels (the balanced schedule when the batch
    fills the device), the other block through the prefill kernel, each kernel
    reading its rows of ``q`` and writing its rows of the output in place. A
    one-token row is a decode: it attends its whole history, as the prefill
    kernel would. ``new_kv`` (the step's rows, not yet written): the prefill
    launch writes every row, the decode rows' included, and runs first.
    Returns ``q``'s shape."""
    b, sq, hq, d = q.shape
    qf = q.reshape(b * sq, hq, d)
    out = torch.empty_like(qf)
    (d0, d1), (p0, p1) = split.dec_range, split.pre_range
    if new_kv is not None and p1 <= p0:
        pool.write(layer_idx, *new_kv)
        new_kv = None
    if new_kv is not None:
        _prefill(qf[p0:p1].unsqueeze(0), pool, layer_idx, split.pre_tables, split.pre_cu, split.pre_q_start,
                 split.pre_max_q, split, scale, err, out=out[p0:p1], new_kv=new_kv, src_row0=p0)
    _decode(qf[d0:d1].unsqueeze(1), pool, layer_idx, split.dec_tables, split.dec_ctx, split, scale, err,
            out=out[d0:d1])
    if new_kv is None and p1 > p0:
        _prefill(qf[p0:p1].unsqueeze(0), pool, layer_idx, split.pre_tables, split.pre_cu, split.pre_q_start,
                 split.pre_max_q, split, scale, err, out=out[p0:p1])
    return out.view(b, sq, hq, d)


def _fusable(pool, layer_idx: int, new_kv: tuple) -> bool:
    """Whether ``ir_paged_prefill`` can take the step's write: this package's
    pool (the kernels address its layers), write slots present, rows of the
    pool's dtype in 16-byte-aligned pieces."""
    k, v, slots = new_kv
    if slots is None or not hasattr(pool, "reference_varlen_form") or not torch.is_tensor(slots):
        return False
    kc = pool.k[layer_idx]
    if k.dtype != kc.dtype or v.dtype != kc.dtype or kc.dtype not in (torch.bfloat16, torch.float16):
        return False
    if slots.dtype != torch.int64 or slots.dim() != 1 or slots.shape[0] != k.shape[0]:
        return False
    return all(t.stride(-1) == 1 and t.stride(0) % 8 == 0 and t.stride(1) % 8 == 0 and t.data_ptr() % 16 == 0
               for t in (k, v))


def _prefill(q, pool, layer_idx: int, block_tables, cu_seqlens_q, q_start, max_q: int, holder, scale: float,
             err, out: torch.Tensor | None = None, new_kv: tuple | None = None, src_row0: int = 0) -> torch.Tensor:
    """Packed query chunks over block tables: the chunked-prefill kernel with
    the step's work plan (built by the first layer, cached on ``holder``) and,
    given ``new_kv``, the step's K/V write in the same launch (``q``'s rows are
    rows ``src_row0..`` of it). Returns ``q``'s shape."""
    b, sq, hq, d = q.shape
    h_kv = pool.k.shape[-2]
    nseq = q_start.shape[0]
    plan = getattr(holder, "prefill_plan", None)
    if plan is not None and plan.f32 != (q.dtype == torch.float32):
        plan = None  # (a plan of the other kind: rebuilt below and kept)
    if plan is None and kernels.prefill_plan_pays(
            nseq, max_q, hq, h_kv, q.device, max_keys=block_tables.shape[1] * pool.block_size, dtype=q.dtype):
        plan = kernels.prefill_plan(
            cu_seqlens_q, q_start, block_tables, b * sq, max_q, pool.block_size, hq, h_kv, d, dtype=q.dtype
        )
        try:
            holder.prefill_plan = plan
        except AttributeError:  # a context object without the field keeps none
            pass
    return kernels.paged_prefill(
        q.reshape(b * sq, hq, d), pool.k[layer_idx], pool.v[layer_idx], block_tables, cu_seqlens_q, q_start, max_q,
        pool.block_size, scale, out=out, err_flags=err, plan=plan, new_kv=new_kv, src_row0=src_row0,
    ).view(b, sq, hq, d)


def _decode(q, pool, layer_idx: int, block_tables, context_lens, holder, scale: float, err,
            out: torch.Tensor | None = None) -> torch.Tensor:
    """One-token decode over block tables: the balanced plan when the batch fills
    the device (cached on ``holder.decode_plan`` for the step's other layers),
    else the fixed split-KV partitions. Returns ``[B, 1, H_q, D]``."""
    b, _, hq, d = q.shape
    h_kv = pool.k.shape[-2]
    k_layer, v_layer = pool.k[layer_idx], pool.v[layer_idx]
    max_blocks = block_tables.shape[1]
    if hasattr(pool, "plan_buffer") and kernels.decode_plan_pays(b, hq, h_kv, max_blocks, pool.block_size, q.device):
        # balanced schedule: built by the step's first layer, reused by the
        # rest -- unless another context's plan has since taken the pool's
        # plan buffer (two decode contexts run interleaved), then rebuilt.
        # Consecutive sequences whose tables share prefix blocks (the prefix
        # cache's reuse) run as pairs, reading those blocks once.
        # A form recorded under graph capture (``gate`` set) plans into its own
        # buffer, which its graph's replays rebuild, and holds it.
        own = getattr(holder, "gate", None) is not None
        plan = holder.decode_plan
        if plan is None or (not own and getattr(pool, "plan_owner", plan) is not plan):
            plan_bytes = kernels.decode_plan_bytes(b, hq, h_kv, max_blocks, pool.block_size)
            if own:
                buf = torch.empty(plan_bytes, dtype=torch.uint8, device=q.device)
                holder.plan_buf = buf
            else:
                buf = pool.plan_buffer(plan_bytes)
            plan = kernels.decode_plan(
                block_tables, context_lens, hq, k_layer, pool.block_size,
                buf=buf, err_flags=err, share_groups=True,
            )
            holder.decode_plan = plan
            if not own:
                pool.plan_owner = plan
        ws = pool.workspace(kernels.planned_workspace_bytes(b, hq, h_kv, d))
        ctr = pool.decode_counters(kernels.decode_num_counters(b, hq, h_kv))
        if own:
            _hold(holder, ws, ctr)
        out = kernels.paged_decode_planned(
            q.reshape(b, hq, d), k_layer, v_layer, plan, scale, out=out, workspace=ws, err_flags=err, counters=ctr
        )
    else:
        ws = ctr = None
        if hasattr(pool, "workspace"):
            need = kernels.decode_workspace_bytes(b, hq, h_kv, d, max_blocks, pool.block_size)
            if need > 0:
                ws = pool.workspace(need)
                ctr = pool.decode_counters(kernels.decode_num_counters(b, hq, h_kv))
        if ws is not None and getattr(holder, "gate", None) is not None:
            _hold(holder, ws, ctr)
        out = kernels.paged_decode(
            q.reshape(b, hq, d), k_layer, v_layer, block_tables, context_lens,
            pool.block_size, scale, out=out, workspace=ws, err_flags=err, counters=ctr,
        )
    return out.view(b, 1, hq, d)



def _hold(holder, *tensors: torch.Tensor) -> None:
    """Keeps pool buffers a captured graph addresses alive with its form (the
    pool may replace them when a later call needs more)."""
    for t in tensors:
        if not any(h is t for h in holder.held):
            holder.held.append(t)
