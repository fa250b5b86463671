"""The reference's own graph decode, unchanged, over this seam.

``CudaGraphDecoder`` (``infrared/engine/cuda_graph.py:170-287``) warms its
decode forward up three times on a side stream over static ``gather_slots`` /
``mask`` buffers, captures it with ``torch.cuda.graph`` into one memory pool
shared by every bucket, and for each later step ``copy_``s the step's
metadata into those buffers and replays. Its ``PagedContext`` has no
block-table fields, so the seam sees only the reference decode metadata.

Under capture the seam records the decode-form check and gates, on the
device, a block-table decode and a mask kernel after it, so each replay takes
the path its own metadata allows. These tests drive exactly that flow (the
decoder's capture steps, restated) and check every replay bit for bit
against an eager call of the same step:

- in the decode form, against the block-table context's output (the
  block-table kernels ran: the mask kernel's rounding differs);
- outside it (a hole in the mask), against the mask kernel's output;
- after the pool's decode buffers were replaced and other allocations were
  made, still equal (the captured form holds what its replays read).
"""

from __future__ import annotations

import gc
from dataclasses import dataclass

import pytest
import torch

from infrared_amd import PagedContext, PagedKVPool, kernels, paged_attention
from infrared_amd.hip_graph import build_decode_static_inputs
from oracle import naive as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
BS, H_KV, N_REP, D, LAYERS = 16, 4, 7, 128, 3
SCALE = D**-0.5


@dataclass(slots=True)
class _ReferenceContext:
    """The reference's PagedContext shape (infrared/cache/paged_kv_cache.py:75-91)."""

    pool: PagedKVPool
    write_slots: torch.Tensor
    gather_slots: torch.Tensor
    use_triton: bool = True


@dataclass(slots=True)
class _Static:
    """One bucket's static buffers: the reference's DecodeInputs metadata plus
    the per-layer q/k/v a model's projections would produce."""

    write_slots: torch.Tensor
    gather_slots: torch.Tensor
    mask: torch.Tensor
    q: torch.Tensor  # [L, B, 1, H_q, D]
    k: torch.Tensor  # [L, B, 1, H_kv, D]
    v: torch.Tensor


def _forward(pool: PagedKVPool, buf: _Static) -> torch.Tensor:
    """The attention part of the captured decode forward, layer by layer
    through the reference seam (infrared/model/layers.py:178-180)."""
    ctx = _ReferenceContext(pool, buf.write_slots, buf.gather_slots)
    outs = [paged_attention(buf.q[l], buf.k[l], buf.v[l], ctx, buf.mask, l, SCALE, N_REP) for l in range(LAYERS)]
    return torch.stack(outs)


def _capture(pool: PagedKVPool, buf: _Static, mempool):
    """CudaGraphDecoder._capture (infrared/engine/cuda_graph.py:263-285):
    three warm-ups on a side stream, then capture into the shared pool."""
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(3):
            _forward(pool, buf)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with (torch.cuda.graph(graph) if mempool is None else torch.cuda.graph(graph, pool=mempool)):
        out = _forward(pool, buf)
    return graph, out


class _Engine:
    """Sequences growing one token per step, with the reference's decode
    metadata for a bucket (pad rows repeat row 0)."""

    def __init__(self, num_seqs: int, bucket: int, t_max: int, first_block: int, seed: int):
        g = torch.Generator().manual_seed(seed)
        self.bucket, self.t_max = bucket, t_max
        nb = t_max // BS
        perm = (torch.randperm(num_seqs * nb, generator=g) + first_block).tolist()
        self.tables = [perm[i * nb : (i + 1) * nb] for i in range(num_seqs)]
        self.num_cached = [int(x) for x in torch.randint(0, t_max - 8, (num_seqs,), generator=g)]
        self.dgen = torch.Generator(device=DEV).manual_seed(seed)

    def step(self) -> _Static:
        inp = build_decode_static_inputs(self.tables, self.num_cached, [0] * len(self.tables), self.bucket,
                                         self.t_max, BS, DEV, torch.bfloat16)
        self.last = inp
        b, hq = self.bucket, H_KV * N_REP
        q = torch.randn(LAYERS, b, 1, hq, D, generator=self.dgen, device=DEV).bfloat16()
        k = torch.randn(LAYERS, b, 1, H_KV, D, generator=self.dgen, device=DEV).bfloat16()
        v = torch.randn(LAYERS, b, 1, H_KV, D, generator=self.dgen, device=DEV).bfloat16()
        # pad rows write row 0's own K/V to row 0's slot (idempotent, as the reference pads)
        n = len(self.tables)
        k[:, n:] = k[:, :1]
        v[:, n:] = v[:, :1]
        self.num_cached = [c + 1 for c in self.num_cached]
        return _Static(inp.write_slots, inp.gather_slots, inp.mask, q, k, v)


def _copy(dst: _Static, src: _Static) -> None:
    for name in _Static.__slots__:
        getattr(dst, name).copy_(getattr(src, name))


def _eager_block_tables(pool: PagedKVPool, eng: _Engine, src: _Static) -> torch.Tensor:
    """The same step through this package's block-table context (fresh tensors)."""
    ctx = PagedContext(pool, src.write_slots.clone(), src.gather_slots.clone(), True,
                       eng.last.block_tables.clone(), eng.last.context_lens.clone())
    return torch.stack([paged_attention(src.q[l], src.k[l], src.v[l], ctx, None, l, SCALE, N_REP)
                        for l in range(LAYERS)])


def _eager_mask_kernel(pool: PagedKVPool, src: _Static) -> torch.Tensor:
    return torch.stack([kernels.paged_attention_masked(src.q[l], pool.k[l], pool.v[l], src.gather_slots, src.mask,
                                                       SCALE) for l in range(LAYERS)])


def test_reference_graph_decoder_replays_on_the_block_table_kernels():
    print("reference graph decode: buckets 64 (planned) and 4 (fixed partitions)", flush=True)
    t_max = 2048
    pool = PagedKVPool(LAYERS, 70 * (t_max // BS), BS, H_KV, D, torch.bfloat16, device=DEV)
    pool.k.normal_()
    pool.v.normal_()
    engines = {64: _Engine(60, 64, t_max, 0, 5), 4: _Engine(3, 4, 1024, 64 * (t_max // BS), 6)}
    assert kernels.decode_plan_pays(64, H_KV * N_REP, H_KV, t_max // BS, BS)
    assert not kernels.decode_plan_pays(4, H_KV * N_REP, H_KV, 1024 // BS, BS)
    graphs, mempool = {}, None
    for step in range(4):
        for bucket in (64, 4):  # the larger bucket first: the smaller one's warm-up then regrows nothing
            eng = engines[bucket]
            src = eng.step()
            if bucket not in graphs:
                buf = _Static(*(getattr(src, n).clone() for n in _Static.__slots__))
                graph, out = _capture(pool, buf, mempool)
                mempool = graph.pool() if mempool is None else mempool
                graphs[bucket] = (graph, buf, out)
            graph, buf, out = graphs[bucket]
            _copy(buf, src)
            if step == 2 and bucket == 64:
                # a hole inside one row's context: not the decode form
                buf.mask[5, 0, 0, 3] = torch.finfo(torch.bfloat16).min
                src.mask[5, 0, 0, 3] = torch.finfo(torch.bfloat16).min
            graph.replay()
            torch.cuda.synchronize()
            got = out.clone()
            if step == 2 and bucket == 64:
                want = _eager_mask_kernel(pool, src)
                assert torch.equal(got, want), f"step {step} bucket {bucket}: replay != mask kernel"
                expect = O.paged_attention_naive(src.q[0, :8].float().cpu(), pool.k[0].float().cpu(),
                                                 pool.v[0].float().cpu(), src.gather_slots[:8].cpu(),
                                                 src.mask[:8].float().cpu(), SCALE, N_REP)
            else:
                want = _eager_block_tables(pool, eng, src)
                torch.cuda.synchronize()
                assert torch.equal(got, want), f"step {step} bucket {bucket}: replay != block-table decode"
                assert not torch.equal(got, _eager_mask_kernel(pool, src)), "the mask kernel's rounding differs"
                expect = O.decode_reference(src.q[0, :8, 0].cpu(), pool.k[0].cpu(), pool.v[0].cpu(),
                                            eng.last.block_tables[:8].cpu(), eng.last.context_lens[:8].cpu(), BS,
                                            SCALE).unsqueeze(1)
            assert (got[0, :8].float().cpu() - expect).abs().max().item() <= 2e-2
            print(f"step {step} bucket {bucket}: ok", flush=True)
        if step == 1:
            # replace the pool's decode buffers and churn the allocator: the
            # graphs must still read live memory
            pool._workspace = pool._counters = pool._plan_buf = None
            pool._ref_form = None
            gc.collect()
            junk = [torch.full((1 << 20,), 7, dtype=torch.int32, device=DEV) for _ in range(8)]
            del junk
    assert pool.err_flags.item() == 0
    assert len(pool._captured_forms) == 2


def test_captured_forms_go_with_their_static_buffers():
    """A captured form lives as long as the gather_slots tensor it was recorded
    for: dropping the graph and its static buffers releases it."""
    t_max = 512
    pool = PagedKVPool(LAYERS, 8 * (t_max // BS), BS, H_KV, D, torch.bfloat16, device=DEV)
    eng = _Engine(8, 8, t_max, 0, 9)
    src = eng.step()
    buf = _Static(*(getattr(src, n).clone() for n in _Static.__slots__))
    graph, out = _capture(pool, buf, None)
    assert len(pool._captured_forms) == 1
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, _eager_block_tables(pool, eng, src))
    del graph, buf, out
    gc.collect()
    assert len(pool._captured_forms) == 0
