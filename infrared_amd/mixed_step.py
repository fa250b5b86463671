"""One engine step of a mixed batch (decode rows + prefill chunks) over every
layer, captured once as a hipGraph and replayed.

The reference's mixed step (``infrared/engine/paged_engine.py:461-516``) packs
all scheduled query tokens into one ``B = 1`` frame and attends with a
quadratic varlen mask (``infrared/model/inputs.py:57-85``) through the paged
seam (``infrared/model/triton_attention.py:81-107``), layer after layer. Here
each layer's attention work is two kernel launches on the step's own
metadata:

1. ``ir_paged_prefill`` for the chunks (causal after their cached prefix),
   whose launch also writes the step's new K/V rows (decode tokens first, then
   the chunk tokens) into the pool at ``write_slots`` -- the K/V write of the
   reference's ``PagedKVPool.write`` -- while its attending workgroups read
   the chunks' own new keys from those rows;
2. the decode of the one-token rows over their block tables: on the balanced
   plan that ``ir_paged_decode_plan`` builds once at the start of the step
   (``ir_paged_decode_planned`` per layer) when the rows fill the device, else
   ``ir_paged_decode``'s fixed split-KV partitions. It follows the prefill,
   which has written its rows' new tokens.

With ``fused=False`` the write is its own launch (``ir_kv_scatter``) ahead of
the decode and then the prefill. With ``overlap=True`` (unfused) the decode
rows' scatter runs first, then the stream forks: the decode (HBM-bound) on
one branch, the chunks' scatter and prefill (MFMA-bound) on the other, joined
before the next layer; captured, they become parallel graph branches (both
streams at the default priority). That measured slower on MI355X at 224
decode rows + 4 x 256-token chunks: 187.5 against 177.5 us per layer, with a
prefill workgroup (~78 KB of LDS) fitting beside each decode workgroup
(72 KB), so the loss is the branches' cost, not CUs held by the prefill.

The per-layer projections around attention are not part of this path; the
caller supplies each layer's q and new K/V (``MixedInputs``).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from infrared_amd import kernels, metadata
from infrared_amd.paged_kv_cache import PagedKVPool


@dataclass(frozen=True)
class MixedConfig:
    name: str
    num_layers: int
    num_decode: int
    decode_ctx_lo: int  # decode context (including the new token) ~ U{lo..hi}
    decode_ctx_hi: int
    num_prefill: int
    chunk: int  # query tokens per prefill chunk
    prefix: int  # cached prefix of every chunk
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    dtype: torch.dtype
    seed: int = 0

    @property
    def scale(self) -> float:
        return self.head_dim**-0.5


MIXED_CONFIGS: dict[str, MixedConfig] = {
    # 224 decode rows (ctx U{256..4096}) + 4 x 256-token prefill chunks, 28 layers
    "qwen7b-mixed": MixedConfig("qwen7b-mixed", 28, 224, 256, 4096, 4, 256, 0, 28, 4, 128, 16, torch.bfloat16, seed=5),
}


@dataclass
class MixedBatch:
    """The step's metadata (fixed for every layer)."""

    write_slots: torch.Tensor  # int64 [num_decode + num_prefill * chunk]
    dec_tables: torch.Tensor  # int32 [num_decode, max_blocks]
    dec_ctx: torch.Tensor  # int32 [num_decode], includes the new token
    pre_tables: torch.Tensor  # int32 [num_prefill, max_blocks]
    cu_seqlens_q: torch.Tensor  # int32 [num_prefill + 1]
    q_start: torch.Tensor  # int32 [num_prefill]
    max_q_len: int


@dataclass
class MixedInputs:
    """Per-layer activations of the step (synthetic in the benchmark)."""

    q_dec: torch.Tensor  # [L, num_decode, H_q, D]
    q_pre: torch.Tensor  # [L, num_prefill * chunk, H_q, D]
    k_new: torch.Tensor  # [L, num_decode + num_prefill * chunk, H_kv, D]
    v_new: torch.Tensor


def make_mixed_case(
    config: str | MixedConfig, device: torch.device | str
) -> tuple[MixedConfig, PagedKVPool, MixedBatch, MixedInputs]:
    """Seeded pool (random history), block tables and step inputs."""
    cfg = MIXED_CONFIGS[config] if isinstance(config, str) else config
    bs = cfg.block_size
    gen = torch.Generator().manual_seed(cfg.seed)
    dec_ctx = torch.randint(cfg.decode_ctx_lo, cfg.decode_ctx_hi + 1, (cfg.num_decode,), generator=gen)
    pre_len = [cfg.prefix + cfg.chunk] * cfg.num_prefill
    nblk = [metadata.blocks_for(int(c), bs) for c in dec_ctx] + [metadata.blocks_for(n, bs) for n in pre_len]
    need = sum(nblk)
    num_blocks = math.ceil(1.25 * need)
    perm = torch.randperm(num_blocks, generator=gen).tolist()
    tables, off = [], 0
    for n in nblk:
        tables.append(perm[off : off + n])
        off += n
    dec_rows, pre_rows = tables[: cfg.num_decode], tables[cfg.num_decode :]
    # new tokens: each decode row's token at position ctx - 1, then each chunk's tokens
    write = [metadata.slot(r, int(c) - 1, bs) for r, c in zip(dec_rows, dec_ctx)]
    for r in pre_rows:
        write += [metadata.slot(r, p, bs) for p in range(cfg.prefix, cfg.prefix + cfg.chunk)]
    cu = [i * cfg.chunk for i in range(cfg.num_prefill + 1)]
    batch = MixedBatch(
        write_slots=torch.tensor(write, dtype=torch.int64, device=device),
        dec_tables=metadata.block_tables_tensor(dec_rows, device),
        dec_ctx=dec_ctx.to(torch.int32).to(device),
        pre_tables=metadata.block_tables_tensor(pre_rows, device),
        cu_seqlens_q=torch.tensor(cu, dtype=torch.int32, device=device),
        q_start=torch.full((cfg.num_prefill,), cfg.prefix, dtype=torch.int32, device=device),
        max_q_len=cfg.chunk,
    )
    pool = PagedKVPool(cfg.num_layers, num_blocks, bs, cfg.num_kv_heads, cfg.head_dim, cfg.dtype, device=device)
    dgen = torch.Generator(device=device).manual_seed(cfg.seed)
    for layer in range(cfg.num_layers):
        pool.k[layer].normal_(generator=dgen)
        pool.v[layer].normal_(generator=dgen)
    L, hq, hkv, d = cfg.num_layers, cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim
    n_new = cfg.num_decode + cfg.num_prefill * cfg.chunk

    def rnd(*shape):
        return torch.randn(*shape, generator=dgen, device=device).to(cfg.dtype)

    inputs = MixedInputs(
        q_dec=rnd(L, cfg.num_decode, hq, d),
        q_pre=rnd(L, cfg.num_prefill * cfg.chunk, hq, d),
        k_new=rnd(L, n_new, hkv, d),
        v_new=rnd(L, n_new, hkv, d),
    )
    return cfg, pool, batch, inputs


class MixedStep:
    """Runs (``eager``) or captures and replays (``replay``) the step over all layers.

    Outputs land in ``out_dec`` ``[L, num_decode, H_q, D]`` and ``out_pre``
    ``[L, num_prefill * chunk, H_q, D]``. The split-KV workspace is allocated
    here once, so a captured graph keeps pointing at live memory.
    """

    def __init__(self, pool: PagedKVPool, batch: MixedBatch, inputs: MixedInputs, scale: float, *,
                 overlap: bool = False, fused: bool = True) -> None:
        self.pool, self.batch, self.inputs, self.scale = pool, batch, inputs, scale
        self.overlap = overlap
        self.fused = fused and not overlap
        dev = pool.device
        self.out_dec = torch.empty_like(inputs.q_dec)
        self.out_pre = torch.empty_like(inputs.q_pre)
        hq, d = inputs.q_dec.shape[2], inputs.q_dec.shape[3]
        nd, max_blocks = batch.dec_tables.shape
        self.planned = kernels.decode_plan_pays(nd, hq, pool.num_kv_heads, max_blocks, pool.block_size, dev)
        if self.planned:
            need = kernels.planned_workspace_bytes(nd, hq, pool.num_kv_heads, d)
            self.plan_buf = torch.empty(
                kernels.decode_plan_bytes(nd, hq, pool.num_kv_heads, max_blocks, pool.block_size),
                dtype=torch.uint8, device=dev,
            )
        else:
            need = kernels.decode_workspace_bytes(nd, hq, pool.num_kv_heads, d, max_blocks, pool.block_size)
            self.plan_buf = None
        self.plan: kernels.DecodePlan | None = None
        npre = batch.q_start.shape[0]
        self.ordered = kernels.prefill_plan_pays(npre, batch.max_q_len, hq, pool.num_kv_heads, dev,
                                                 max_keys=batch.pre_tables.shape[1] * pool.block_size,
                                                 dtype=pool.dtype)
        self.plan_pre_buf = (torch.empty(kernels.prefill_plan_bytes(npre, batch.max_q_len, hq, pool.num_kv_heads, d),
                                         dtype=torch.uint8, device=dev) if self.ordered else None)
        self.plan_pre: kernels.PrefillPlan | None = None
        self.workspace = torch.empty(max(need, 256), dtype=torch.uint8, device=dev) if need > 0 else None
        self.counters = torch.zeros(kernels.decode_num_counters(nd, hq, pool.num_kv_heads), dtype=torch.int32,
                                    device=dev)
        self.err = torch.zeros(1, dtype=torch.int32, device=dev)
        self._side = torch.cuda.Stream(device=dev) if overlap else None
        self._graph: torch.cuda.CUDAGraph | None = None

    def _decode(self, layer: int) -> None:
        b, inp, pool = self.batch, self.inputs, self.pool
        if self.planned:
            kernels.paged_decode_planned(
                inp.q_dec[layer], pool.k[layer], pool.v[layer], self.plan, self.scale, out=self.out_dec[layer],
                workspace=self.workspace, err_flags=self.err, counters=self.counters,
            )
            return
        kernels.paged_decode(
            inp.q_dec[layer], pool.k[layer], pool.v[layer], b.dec_tables, b.dec_ctx, pool.block_size, self.scale,
            out=self.out_dec[layer], workspace=self.workspace, err_flags=self.err, counters=self.counters,
        )

    def _prefill(self, layer: int, fused: bool = False) -> None:
        b, inp, pool = self.batch, self.inputs, self.pool
        kernels.paged_prefill(
            inp.q_pre[layer], pool.k[layer], pool.v[layer], b.pre_tables, b.cu_seqlens_q, b.q_start, b.max_q_len,
            pool.block_size, self.scale, out=self.out_pre[layer], err_flags=self.err, plan=self.plan_pre,
            new_kv=(inp.k_new[layer], inp.v_new[layer], b.write_slots) if fused else None,
            src_row0=inp.q_dec.shape[1],
        )

    def _layer(self, layer: int) -> None:
        b, inp, pool = self.batch, self.inputs, self.pool
        if self.fused:
            # the prefill launch writes every new row (the decode rows' too)
            # and reads the chunks' own keys from them; the decode follows
            self._prefill(layer, fused=True)
            self._decode(layer)
            return
        if self._side is None:
            kernels.kv_scatter(pool.k[layer], pool.v[layer], inp.k_new[layer], inp.v_new[layer], b.write_slots,
                               self.err)
            self._decode(layer)
            self._prefill(layer)
            return
        # the decode rows' new K/V first (the decode reads them), then the
        # chunks' rows and the prefill on the side stream beside the decode
        nd = inp.q_dec.shape[1]
        main = torch.cuda.current_stream(pool.device)
        kernels.kv_scatter(pool.k[layer], pool.v[layer], inp.k_new[layer, :nd], inp.v_new[layer, :nd],
                           b.write_slots[:nd], self.err)
        self._side.wait_stream(main)
        with torch.cuda.stream(self._side):
            kernels.kv_scatter(pool.k[layer], pool.v[layer], inp.k_new[layer, nd:], inp.v_new[layer, nd:],
                               b.write_slots[nd:], self.err)
            self._prefill(layer)
        self._decode(layer)
        main.wait_stream(self._side)  # both are done before the next layer's scatter

    def eager(self) -> None:
        if self.planned:  # one plan for the step's decode rows, shared by every layer
            b = self.batch
            self.plan = kernels.decode_plan(
                b.dec_tables, b.dec_ctx, self.inputs.q_dec.shape[2], self.pool.k[0], self.pool.block_size,
                buf=self.plan_buf, err_flags=self.err,
            )
        if self.ordered:  # one prefill work plan per step, shared by every layer
            b = self.batch
            self.plan_pre = kernels.prefill_plan(
                b.cu_seqlens_q, b.q_start, b.pre_tables, self.inputs.q_pre.shape[1], b.max_q_len,
                self.pool.block_size, self.inputs.q_pre.shape[2], self.pool.num_kv_heads,
                self.inputs.q_pre.shape[3], buf=self.plan_pre_buf, dtype=self.inputs.q_pre.dtype,
            )
        for layer in range(self.pool.num_layers):
            self._layer(layer)

    def capture(self, warmup: int = 1) -> None:
        stream = torch.cuda.Stream(device=self.pool.device)
        stream.wait_stream(torch.cuda.current_stream(self.pool.device))
        with torch.cuda.stream(stream):
            for _ in range(warmup):
                self.eager()
        torch.cuda.current_stream(self.pool.device).wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self.eager()
        self._graph = graph

    def replay(self) -> None:
        if self._graph is None:
            self.capture()
        self._graph.replay()
