"""CPU oracle for the paged-attention hot path — TEST INFRASTRUCTURE ONLY.

A restatement, in plain torch on the CPU, of the reference's naive paged
attention fallback and the metadata that feeds it. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg use it, as the
checker; the product (``infrared_amd``) never imports it.

Restated functions and the reference lines they follow:

- ``pool_write``       infrared/cache/paged_kv_cache.py:48-57 (index_put scatter)
- ``pool_gather``      infrared/cache/paged_kv_cache.py:59-72
- ``repeat_kv``        infrared/model/layers.py:92-99
- ``masked_attention`` infrared/model/layers.py:102-118
- ``paged_attention_naive``  infrared/model/triton_attention.py:110-129
- ``blockwise_attention``    infrared/model/triton_attention.py:135-177
- ``split_kv_attention``     (new) partition + log-sum-exp merge of the same math
- ``slot``             infrared/engine/paged_engine.py:621-625
- ``decode_gather_slots``    infrared/engine/paged_engine.py:306-314
- ``decode_mask``      infrared/engine/paged_engine.py:630-638
- ``attention_mask``   infrared/model/inputs.py:33-54
- ``varlen_mask``      infrared/model/inputs.py:57-85
- ``default_buckets`` / ``pick_bucket``  infrared/engine/cuda_graph.py:58-81
- ``decode_reference`` (new) per-sequence decode over the block tables with no
  padding, in a chosen float dtype; equal to ``paged_attention_naive`` on
  the gather_slots/mask the engine builds (pinned in tests/test_oracle.py).
- ``rotary_cos_sin``   infrared/model/layers.py:121-136 (RotaryEmbedding)
- ``rotate_half`` / ``apply_rotary_pos_emb``  infrared/model/layers.py:72-89
- ``prefill_reference`` (new) per-sequence causal attention of packed query
  chunks after a cached prefix, over the block tables; equal to
  ``paged_attention_naive`` on the prefill metadata of
  infrared/engine/paged_engine.py:194-207 (``attention_mask``) and on the
  packed mixed-step metadata of infrared/engine/paged_engine.py:461-516
  (``varlen_mask``) (pinned in tests/test_oracle.py).

How each is pinned (tests/test_oracle.py): ``masked_attention`` against
torch's SDPA and an fp64 brute force; the streaming/split variants against
the one-shot softmax for many block/partition sizes; metadata against the
reference tests' known-answer values (tests/golden/reference_kats.json);
``decode_reference`` and ``prefill_reference`` against
``paged_attention_naive`` on the engine's metadata and closed forms (one-hot
scores, constant V).
"""

from __future__ import annotations

from collections.abc import Sequence

import torch

# --------------------------------------------------------------------- pool


def pool_write(
    k_layer: torch.Tensor, v_layer: torch.Tensor, k: torch.Tensor, v: torch.Tensor, slots: torch.Tensor
) -> None:
    """``k_layer[slots] = k; v_layer[slots] = v`` (rows ``[N, H_kv, D]``)."""
    k_layer[slots] = k
    v_layer[slots] = v


def pool_gather(
    k_layer: torch.Tensor, v_layer: torch.Tensor, gather_slots: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor]:
    """``[B, T]`` slot ids -> ``[B, T, H_kv, D]`` K and V."""
    b, t = gather_slots.shape
    flat = gather_slots.reshape(-1)
    k = k_layer[flat].reshape(b, t, *k_layer.shape[1:])
    v = v_layer[flat].reshape(b, t, *v_layer.shape[1:])
    return k, v


# --------------------------------------------------------------------- rotary embedding


def rotary_cos_sin(positions: torch.Tensor, head_dim: int, theta: float) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 ``cos``/``sin`` ``[*positions.shape, head_dim]`` for absolute positions."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    freqs = positions.to(torch.float32)[..., None] * inv_freq
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos(), emb.sin()


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rotary_pos_emb(
    q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor]:
    """``q``/``k`` ``[B, S, H, D]``, ``cos``/``sin`` ``[B, S, D]``; tables cast to the
    activation dtype first, then ``x * cos + rotate_half(x) * sin`` in that dtype."""
    cos = cos.unsqueeze(2).to(q.dtype)
    sin = sin.unsqueeze(2).to(q.dtype)
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin


# --------------------------------------------------------------------- math


def repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """``[B, S, H_kv, D]`` -> ``[B, S, H_kv * n_rep, D]``; head ``j`` <- kv head ``j // n_rep``."""
    if n_rep == 1:
        return x
    return x.repeat_interleave(n_rep, dim=2)


def masked_attention(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: torch.Tensor, scale: float
) -> torch.Tensor:
    """Scores in the input dtype plus additive mask, fp32 softmax, cast back, then PV."""
    scores = torch.einsum("bqhd,bkhd->bhqk", q, k) * scale + mask
    attn = torch.softmax(scores.to(torch.float32), dim=-1).to(q.dtype)
    return torch.einsum("bhqk,bkhd->bqhd", attn, v)


def paged_attention_naive(
    q: torch.Tensor,
    k_layer: torch.Tensor,
    v_layer: torch.Tensor,
    gather_slots: torch.Tensor,
    mask: torch.Tensor,
    scale: float,
    n_rep: int,
) -> torch.Tensor:
    """Gather the full padded history, repeat K/V per GQA group, one-shot masked softmax."""
    k_all, v_all = pool_gather(k_layer, v_layer, gather_slots)
    k_all = repeat_kv(k_all, n_rep)
    v_all = repeat_kv(v_all, n_rep)
    return masked_attention(q, k_all, v_all, mask, scale)


def blockwise_attention(
    q: torch.Tensor,
    k_all: torch.Tensor,
    v_all: torch.Tensor,
    mask: torch.Tensor,
    scale: float,
    block_n: int | None = None,
) -> torch.Tensor:
    """Streaming online softmax over key blocks of ``block_n`` (fp32 state)."""
    b, sq, h, d = q.shape
    t = k_all.shape[1]
    block_n = block_n or t
    qh = q.permute(0, 2, 1, 3).to(torch.float32)
    kh = k_all.permute(0, 2, 1, 3).to(torch.float32)
    vh = v_all.permute(0, 2, 1, 3).to(torch.float32)
    m_i = torch.full((b, h, sq, 1), float("-inf"))
    l_i = torch.zeros((b, h, sq, 1))
    acc = torch.zeros((b, h, sq, d))
    for j in range(0, t, block_n):
        qk = (qh @ kh[:, :, j : j + block_n].transpose(-1, -2)) * scale + mask[:, :, :, j : j + block_n]
        m_ij = torch.maximum(m_i, qk.max(dim=-1, keepdim=True).values)
        p = torch.exp(qk - m_ij)
        alpha = torch.exp(m_i - m_ij)
        l_i = l_i * alpha + p.sum(dim=-1, keepdim=True)
        acc = acc * alpha + p @ vh[:, :, j : j + block_n]
        m_i = m_ij
    return (acc / l_i).permute(0, 2, 1, 3).to(q.dtype)


def split_kv_attention(
    q: torch.Tensor,
    k_all: torch.Tensor,
    v_all: torch.Tensor,
    mask: torch.Tensor,
    scale: float,
    part_len: int,
) -> torch.Tensor:
    """Split the key axis into partitions of ``part_len``; each yields (max, sum,
    unnormalised acc); merge with weights exp(m_p - M). fp32 throughout."""
    b, sq, h, d = q.shape
    t = k_all.shape[1]
    qh = q.permute(0, 2, 1, 3).to(torch.float32)
    kh = k_all.permute(0, 2, 1, 3).to(torch.float32)
    vh = v_all.permute(0, 2, 1, 3).to(torch.float32)
    ms, ls, accs = [], [], []
    for j in range(0, t, part_len):
        s = (qh @ kh[:, :, j : j + part_len].transpose(-1, -2)) * scale + mask[:, :, :, j : j + part_len]
        m = s.max(dim=-1, keepdim=True).values
        p = torch.exp(s - m)
        ms.append(m)
        ls.append(p.sum(dim=-1, keepdim=True))
        accs.append(p @ vh[:, :, j : j + part_len])
    big_m = torch.stack(ms).max(dim=0).values
    num = torch.zeros((b, h, sq, d))
    den = torch.zeros((b, h, sq, 1))
    for m, l, acc in zip(ms, ls, accs):
        w = torch.exp(m - big_m)
        num = num + w * acc
        den = den + w * l
    return (num / den).permute(0, 2, 1, 3).to(q.dtype)


# --------------------------------------------------------------------- metadata


def slot(block_table: Sequence[int], pos: int, block_size: int) -> int:
    return block_table[pos // block_size] * block_size + (pos % block_size)


def decode_gather_slots(
    block_tables: Sequence[Sequence[int]], context_lens: Sequence[int], block_size: int, t_max: int
) -> torch.Tensor:
    """``[B, t_max]`` int64, row ``i`` = slots of positions ``[0, ctx_i)``, zeros after."""
    out = torch.zeros(len(block_tables), t_max, dtype=torch.long)
    for i, (bt, n) in enumerate(zip(block_tables, context_lens)):
        bt_t = torch.as_tensor(list(bt), dtype=torch.long)
        pos = torch.arange(n)
        out[i, :n] = bt_t[pos // block_size] * block_size + (pos % block_size)
    return out


def decode_mask(context_lens: Sequence[int], max_len: int, dtype: torch.dtype) -> torch.Tensor:
    cols = torch.arange(max_len)
    lens = torch.tensor(list(context_lens))[:, None]
    invalid = cols[None, :] >= lens
    mask = torch.zeros(len(context_lens), 1, 1, max_len, dtype=dtype)
    return mask.masked_fill(invalid[:, None, None, :], torch.finfo(dtype).min)


def attention_mask(
    pad_lens: Sequence[int], q_start_col: int, q_len: int, total_k: int, dtype: torch.dtype
) -> torch.Tensor:
    q_cols = torch.arange(q_start_col, q_start_col + q_len)
    k_cols = torch.arange(total_k)
    causal = k_cols[None, :] <= q_cols[:, None]
    pad = torch.tensor(list(pad_lens))[:, None]
    key_valid = k_cols[None, :] >= pad
    allowed = causal[None, :, :] & key_valid[:, None, :]
    mask = torch.zeros(len(pad_lens), 1, q_len, total_k, dtype=dtype)
    return mask.masked_fill(~allowed[:, None, :, :], torch.finfo(dtype).min)


def varlen_mask(
    q_seq_ids: torch.Tensor, q_pos: torch.Tensor, k_seq_ids: torch.Tensor, k_pos: torch.Tensor, dtype: torch.dtype
) -> torch.Tensor:
    allowed = (q_seq_ids[:, None] == k_seq_ids[None, :]) & (k_pos[None, :] <= q_pos[:, None])
    mask = torch.zeros(1, 1, q_seq_ids.shape[0], k_seq_ids.shape[0], dtype=dtype)
    return mask.masked_fill(~allowed[None, None, :, :], torch.finfo(dtype).min)


def default_buckets(max_num_seqs: int) -> tuple[int, ...]:
    if max_num_seqs < 1:
        raise ValueError("max_num_seqs must be >= 1")
    buckets, p = [], 1
    while p < max_num_seqs:
        buckets.append(p)
        p *= 2
    buckets.append(max_num_seqs)
    return tuple(buckets)


def pick_bucket(b: int, buckets: tuple[int, ...]) -> int:
    for bucket in buckets:
        if bucket >= b:
            return bucket
    raise ValueError(f"batch size {b} exceeds largest bucket {buckets[-1]}")


# --------------------------------------------------------------------- per-sequence decode


def decode_reference(
    q: torch.Tensor,
    k_layer: torch.Tensor,
    v_layer: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    block_size: int,
    scale: float,
    compute_dtype: torch.dtype = torch.float32,
    seqs: Sequence[int] | None = None,
) -> torch.Tensor:
    """Decode attention per sequence over exactly ``ctx_i`` keys (no padding).

    ``q`` ``[B, H_q, D]``; returns ``[B, H_q, D]`` in ``compute_dtype`` (rows not in
    ``seqs`` are left zero). Context 0 gives a zero row.
    """
    b, hq, d = q.shape
    h_kv = k_layer.shape[1]
    n_rep = hq // h_kv
    out = torch.zeros(b, hq, d, dtype=compute_dtype)
    bt = block_tables.cpu().long()
    cl = context_lens.cpu().long()
    for i in range(b) if seqs is None else seqs:
        n = int(cl[i])
        if n == 0:
            continue
        pos = torch.arange(n)
        slots = bt[i, pos // block_size] * block_size + pos % block_size
        k = k_layer[slots].to(compute_dtype)  # [n, H_kv, D]
        v = v_layer[slots].to(compute_dtype)
        qi = q[i].to(compute_dtype).reshape(h_kv, n_rep, d)
        s = torch.einsum("grd,ngd->grn", qi, k) * scale
        p = torch.softmax(s, dim=-1)
        out[i] = torch.einsum("grn,ngd->grd", p, v).reshape(hq, d)
    return out


# --------------------------------------------------------------------- per-sequence prefill


def prefill_reference(
    q: torch.Tensor,
    k_layer: torch.Tensor,
    v_layer: torch.Tensor,
    block_tables: torch.Tensor,
    cu_seqlens_q: Sequence[int] | torch.Tensor,
    q_start: Sequence[int] | torch.Tensor,
    block_size: int,
    scale: float,
    compute_dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """Causal attention of packed query chunks over the block tables.

    ``q`` ``[total_q, H_q, D]``; sequence ``b`` owns rows
    ``cu_seqlens_q[b]:cu_seqlens_q[b+1]``, whose query ``i`` is at position
    ``q_start[b] + i`` and attends keys ``0 .. q_start[b] + i`` of the sequence.
    Returns ``[total_q, H_q, D]`` in ``compute_dtype``.
    """
    total_q, hq, d = q.shape
    h_kv = k_layer.shape[1]
    n_rep = hq // h_kv
    cu = [int(x) for x in (cu_seqlens_q.tolist() if torch.is_tensor(cu_seqlens_q) else cu_seqlens_q)]
    qs = [int(x) for x in (q_start.tolist() if torch.is_tensor(q_start) else q_start)]
    bt = block_tables.cpu().long()
    out = torch.zeros(total_q, hq, d, dtype=compute_dtype)
    for b in range(len(qs)):
        lo, hi = cu[b], cu[b + 1]
        if hi <= lo:
            continue
        n_keys = qs[b] + (hi - lo)
        pos = torch.arange(n_keys)
        slots = bt[b, pos // block_size] * block_size + pos % block_size
        k = k_layer[slots].to(compute_dtype)  # [n_keys, H_kv, D]
        v = v_layer[slots].to(compute_dtype)
        qb = q[lo:hi].to(compute_dtype).reshape(hi - lo, h_kv, n_rep, d)
        s = torch.einsum("igrd,ngd->grin", qb, k) * scale
        q_pos = qs[b] + torch.arange(hi - lo)
        allowed = pos[None, :] <= q_pos[:, None]  # [i, n]
        s = s.masked_fill(~allowed, float("-inf"))
        p = torch.softmax(s, dim=-1)
        out[lo:hi] = torch.einsum("grin,ngd->igrd", p, v).reshape(hi - lo, hq, d)
    return out
