"""hipGraph capture/replay of the decode step (replaces ``infrared/engine/cuda_graph.py``).

Same API as the reference module:

- ``default_buckets`` / ``pick_bucket`` (``infrared/engine/cuda_graph.py:58-81``);
- ``build_decode_static_inputs`` (``:105-155``): fixed-shape inputs for a batch
  bucket, pad-by-repeating row 0, key axis padded to ``t_max``. Built
  vectorised on the device instead of a Python loop over ``B * ctx`` tokens, and
  carrying the ``block_tables``/``context_lens`` the HIP decode kernel reads;
- ``HipGraphDecoder`` (in place of ``CudaGraphDecoder``, ``:170-287``): one
  captured graph per bucket sharing one memory pool; ``decode()`` copies the
  step's metadata into the static buffers and replays.

PyTorch-ROCm's ``torch.cuda.CUDAGraph`` is a hipGraph; the HIP kernels are
launched on torch's current stream, so they are captured as graph kernel
nodes. They neither synchronise nor allocate. The pool's decode buffers
(split-KV workspace, arrival counters, plan buffer) are grown during a
bucket's warm-up, outside capture; a larger bucket captured later may grow
them again, which replaces the pool's tensors, so every captured graph keeps
references to the buffers it was captured with and its replays stay on that
live memory. The kernel reads only ``context_lens[b]`` keys per row, so a
replay costs the real context, not ``t_max``.
"""

from __future__ import annotations

from collections.abc import Callable, Sequence
from dataclasses import dataclass

import torch

from infrared_amd import metadata
from infrared_amd.paged_kv_cache import PagedContext, PagedKVPool


def default_buckets(max_num_seqs: int) -> tuple[int, ...]:
    """Powers of two below ``max_num_seqs``, then ``max_num_seqs`` itself."""
    if max_num_seqs < 1:
        raise ValueError("max_num_seqs must be >= 1")
    out: list[int] = []
    p = 1
    while p < max_num_seqs:
        out.append(p)
        p *= 2
    out.append(max_num_seqs)
    return tuple(out)


def pick_bucket(b: int, buckets: tuple[int, ...]) -> int:
    """Smallest bucket ``>= b``; raises ``ValueError`` past the largest."""
    for bucket in buckets:
        if bucket >= b:
            return bucket
    raise ValueError(f"batch size {b} exceeds largest bucket {buckets[-1]}")


@dataclass(slots=True)
class DecodeInputs:
    """Fixed-shape decode inputs for bucket ``B`` and key axis ``t_max``.

    ``ids`` ``[B, 1]``, ``positions`` ``[B, 1]``, ``write_slots`` ``[B]``,
    ``gather_slots`` ``[B, t_max]``, ``mask`` ``[B, 1, 1, t_max]`` (the
    reference fields), plus ``block_tables`` ``[B, ceil(t_max / bs)]`` int32 and
    ``context_lens`` ``[B]`` int32.
    """

    ids: torch.Tensor
    positions: torch.Tensor
    write_slots: torch.Tensor
    gather_slots: torch.Tensor
    mask: torch.Tensor
    block_tables: torch.Tensor
    context_lens: torch.Tensor


def build_decode_static_inputs(
    block_tables: Sequence[Sequence[int]],
    num_cached: Sequence[int],
    last_tokens: Sequence[int],
    bucket_b: int,
    t_max: int,
    block_size: int,
    device: torch.device | str,
    dtype: torch.dtype,
) -> DecodeInputs:
    """One decode step's inputs at fixed ``(bucket_b, t_max)``; rows ``[b:]`` repeat row 0.

    Row ``i``'s new token is at position ``num_cached[i]`` (written to
    ``slot(bt_i, num_cached[i])``) and attends ``[0, num_cached[i]]``.
    """
    b = len(last_tokens)
    if not 0 < b <= bucket_b:
        raise ValueError(f"need 0 < b ({b}) <= bucket_b ({bucket_b})")
    width = metadata.blocks_for(t_max, block_size)
    rows = [i if i < b else 0 for i in range(bucket_b)]
    ctx = [num_cached[j] + 1 for j in rows]
    for c in ctx:
        if c > t_max:
            raise ValueError(f"context_len {c} exceeds t_max {t_max}")
    bt = metadata.block_tables_tensor(
        [list(block_tables[j])[:width] for j in rows], device, width
    )
    cl = torch.tensor(ctx, dtype=torch.int32, device=device)
    nc = torch.tensor([num_cached[j] for j in rows], dtype=torch.long, device=device)
    ids = torch.tensor([[last_tokens[j]] for j in rows], dtype=torch.long, device=device)
    return DecodeInputs(
        ids=ids,
        positions=nc[:, None].clone(),
        write_slots=metadata.decode_write_slots(bt, nc, block_size),
        gather_slots=metadata.gather_slots_from_tables(bt, cl, block_size, t_max),
        mask=metadata.decode_mask(cl, t_max, dtype),
        block_tables=bt,
        context_lens=cl,
    )


@dataclass(slots=True)
class _Captured:
    graph: torch.cuda.CUDAGraph
    buf: DecodeInputs
    out: torch.Tensor
    # the pool buffers the graph's kernels address (kept alive for its replays)
    pool_buffers: tuple


class HipGraphDecoder:
    """Per-bucket hipGraph decode: capture once per bucket, then replay each step.

    ``model`` is anything with the reference model's call
    ``forward(ids, positions, mask, paged=PagedContext)`` returning
    ``[B, 1, vocab]``-like output (the last position is taken), or a plain
    callable ``fn(DecodeInputs, PagedContext) -> Tensor`` passed as
    ``step_fn``. Replays must not overlap (they share one memory pool).
    """

    def __init__(
        self,
        model,
        pool: PagedKVPool,
        *,
        max_num_seqs: int,
        t_max: int,
        block_size: int,
        use_triton: bool = True,
        warmup_steps: int = 3,
        step_fn: Callable[[DecodeInputs, PagedContext], torch.Tensor] | None = None,
    ) -> None:
        self.model = model
        self.pool = pool
        self.buckets = default_buckets(max_num_seqs)
        self.t_max = t_max
        self.block_size = block_size
        self.use_triton = use_triton
        self.warmup_steps = warmup_steps
        self.step_fn = step_fn
        self.device = pool.device
        self.dtype = pool.dtype
        self._graphs: dict[int, _Captured] = {}
        self._mempool = None

    def decode(
        self,
        block_tables: Sequence[Sequence[int]],
        num_cached: Sequence[int],
        last_tokens: Sequence[int],
    ) -> torch.Tensor:
        """Advance the running set one token by graph replay; returns the first ``b`` rows."""
        b = len(last_tokens)
        bucket = pick_bucket(b, self.buckets)
        inp = build_decode_static_inputs(
            block_tables, num_cached, last_tokens, bucket, self.t_max, self.block_size,
            self.device, self.dtype,
        )
        if bucket not in self._graphs:
            self._capture(bucket, inp)
        else:
            self._copy_inputs(self._graphs[bucket].buf, inp)
        self._graphs[bucket].graph.replay()
        return self._graphs[bucket].out[:b]

    def _context(self, buf: DecodeInputs) -> PagedContext:
        return PagedContext(
            self.pool, buf.write_slots, buf.gather_slots, self.use_triton, buf.block_tables,
            buf.context_lens,
        )

    def _forward(self, buf: DecodeInputs) -> torch.Tensor:
        paged = self._context(buf)
        if self.step_fn is not None:
            return self.step_fn(buf, paged)
        logits = self.model.forward(buf.ids, buf.positions, buf.mask, paged=paged)
        return logits[:, -1]

    @staticmethod
    def _copy_inputs(dst: DecodeInputs, src: DecodeInputs) -> None:
        for name in DecodeInputs.__slots__:
            getattr(dst, name).copy_(getattr(src, name))

    def _capture(self, bucket: int, inp: DecodeInputs) -> None:
        buf = DecodeInputs(*(getattr(inp, n).clone() for n in DecodeInputs.__slots__))
        stream = torch.cuda.Stream(device=self.device)
        stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(stream):
            for _ in range(self.warmup_steps):
                self._forward(buf)
        torch.cuda.current_stream(self.device).wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        ctx = (
            torch.cuda.graph(graph)
            if self._mempool is None
            else torch.cuda.graph(graph, pool=self._mempool)
        )
        with ctx:
            out = self._forward(buf)
        if self._mempool is None:
            self._mempool = graph.pool()
        held = tuple(getattr(self.pool, n, None) for n in ("_workspace", "_counters", "_plan_buf"))
        self._graphs[bucket] = _Captured(graph=graph, buf=buf, out=out, pool_buffers=held)
