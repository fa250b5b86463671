"""Seeded synthetic paged-attention workloads at the benchmark shapes.

Decode workloads (one query token per sequence):

- ``qwen0.5b-fp32``: 8 seqs, 14 q / 2 kv heads, head_dim 64, block 16, fp32,
  context U{1..512}, pool of 512 blocks, scale 1/8.
- ``qwen7b-bf16``: 64 seqs, 28 q / 4 kv heads, head_dim 128, block 16, bf16,
  context U{512..4096}, pool 1.25x the blocks needed.
- ``qwen7b-skewed``: 16 seqs, 28/4 heads, head_dim 128, bf16, context
  round(lognormal(8, 1.2)) clipped to [16, 32768], pool 1.25x.
- ``qwen7b-pairs``: ``qwen7b-bf16`` where sequences 2i and 2i+1 share the
  block ids of the first half of the shorter context (whole blocks) -- a
  cached prompt prefix the prefix cache hands both (parallel samples, a
  common system prompt); the rest of each context is private.

Prefill workload (``make_prefill_case``):

- ``qwen7b-prefill``: 8 sequences, each a 512-token chunk after a cached
  prefix of U{0..8192} tokens drawn per sequence; sequences 2i and 2i+1 share
  the block ids of the full blocks of their common prefix (prefix caching
  shares full blocks; a partial last block stays private), 28 q / 4 kv heads,
  head_dim 128, block 16, bf16, pool 1.25x the distinct blocks needed.

Each sequence's block table is a consecutive chunk of one random permutation
of the pool's block ids (non-contiguous physical blocks). q and the whole K/V
pool are N(0, 1) drawn in fp32 and cast to the workload dtype. Metadata is
drawn on the CPU from ``torch.Generator(seed)``; q/K/V are drawn on the target
device from a generator with the same seed. ``rotations > 1`` lays out that
many disjoint copies of the block tables over one larger pool (each with its
own K/V values) so back-to-back calls can walk different memory. The K/V
layer tensors are ``[num_slots, H_kv, D]`` views of head-major storage
``[H_kv, num_slots, D]`` by default (``layout="slot_major"`` gives the
contiguous reference layout).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class DecodeConfig:
    name: str
    num_seqs: int
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    dtype: torch.dtype
    ctx_kind: str  # "uniform" | "lognormal"
    ctx_lo: int
    ctx_hi: int
    pool_blocks: int | None = None  # None: ceil(1.25 * blocks needed)
    lognormal_mu: float = 0.0
    lognormal_sigma: float = 1.0
    seed: int = 0
    pair_share: float = 0.0  # sequences 2i, 2i+1 share this fraction of the shorter context (whole blocks)

    @property
    def n_rep(self) -> int:
        return self.num_q_heads // self.num_kv_heads

    @property
    def scale(self) -> float:
        return self.head_dim**-0.5


DECODE_CONFIGS: dict[str, DecodeConfig] = {
    "qwen0.5b-fp32": DecodeConfig(
        "qwen0.5b-fp32", 8, 14, 2, 64, 16, torch.float32, "uniform", 1, 512, pool_blocks=512, seed=1
    ),
    "qwen7b-bf16": DecodeConfig(
        "qwen7b-bf16", 64, 28, 4, 128, 16, torch.bfloat16, "uniform", 512, 4096, seed=2
    ),
    "qwen7b-skewed": DecodeConfig(
        "qwen7b-skewed", 16, 28, 4, 128, 16, torch.bfloat16, "lognormal", 16, 32768,
        lognormal_mu=8.0, lognormal_sigma=1.2, seed=3,
    ),
    "qwen7b-pairs": DecodeConfig(
        "qwen7b-pairs", 64, 28, 4, 128, 16, torch.bfloat16, "uniform", 512, 4096, seed=2, pair_share=0.5
    ),
}


@dataclass
class DecodeCase:
    config: DecodeConfig
    q: torch.Tensor  # [B, H_q, D]
    k_cache: torch.Tensor  # [num_slots, H_kv, D] (one layer)
    v_cache: torch.Tensor
    block_tables: list[torch.Tensor]  # per rotation, int32 [B, max_blocks]
    context_lens: torch.Tensor  # int32 [B]
    pool_blocks: int  # blocks per rotation

    @property
    def block_size(self) -> int:
        return self.config.block_size

    @property
    def kv_bytes(self) -> int:
        """Algorithmic K+V bytes one call reads: sum(ctx) * 2 * H_kv * D * sizeof."""
        c = self.config
        esize = torch.tensor([], dtype=c.dtype).element_size()
        return int(self.context_lens.long().sum()) * 2 * c.num_kv_heads * c.head_dim * esize

    @property
    def shared_tokens(self) -> int:
        """Tokens the second sequence of each sharing pair reads from the
        first one's blocks (whole shared blocks inside both contexts)."""
        if self.config.pair_share <= 0:
            return 0
        bs, bt, ctx = self.config.block_size, self.block_tables[0].cpu(), self.context_lens.cpu().tolist()
        n = 0
        for i in range(0, len(ctx) - 1, 2):
            full = min(ctx[i], ctx[i + 1]) // bs
            j = 0
            while j < full and int(bt[i, j]) == int(bt[i + 1, j]):
                j += 1
            n += j * bs
        return n

    @property
    def unique_kv_bytes(self) -> int:
        """K+V bytes of the distinct keys: shared prefix blocks counted once."""
        c = self.config
        esize = torch.tensor([], dtype=c.dtype).element_size()
        return (int(self.context_lens.long().sum()) - self.shared_tokens) * 2 * c.num_kv_heads * c.head_dim * esize


def context_lengths(cfg: DecodeConfig, gen: torch.Generator) -> torch.Tensor:
    if cfg.ctx_kind == "uniform":
        return torch.randint(cfg.ctx_lo, cfg.ctx_hi + 1, (cfg.num_seqs,), generator=gen)
    x = torch.empty(cfg.num_seqs, dtype=torch.float64).log_normal_(
        cfg.lognormal_mu, cfg.lognormal_sigma, generator=gen
    )
    return torch.clamp(torch.round(x), cfg.ctx_lo, cfg.ctx_hi).long()


def make_decode_case(
    config: str | DecodeConfig,
    device: torch.device | str,
    *,
    seed: int | None = None,
    rotations: int = 1,
    num_seqs: int | None = None,
    layout: str = "head_major",
) -> DecodeCase:
    cfg = DECODE_CONFIGS[config] if isinstance(config, str) else config
    if num_seqs is not None:
        cfg = DecodeConfig(**{**cfg.__dict__, "num_seqs": num_seqs})
    seed = cfg.seed if seed is None else seed
    gen = torch.Generator().manual_seed(seed)
    bs = cfg.block_size
    ctx = context_lengths(cfg, gen)
    nblk = (ctx + bs - 1) // bs
    need = int(nblk.sum())
    pool_blocks = cfg.pool_blocks or math.ceil(1.25 * need)
    if pool_blocks < need:
        raise ValueError(f"{cfg.name}: pool of {pool_blocks} blocks < {need} needed")
    width = int(nblk.max())
    tables = []
    for r in range(rotations):
        perm = torch.randperm(pool_blocks, generator=gen) + r * pool_blocks
        bt = torch.zeros(cfg.num_seqs, width, dtype=torch.int32)
        off = 0
        for i, n in enumerate(nblk.tolist()):
            bt[i, :n] = perm[off : off + n].to(torch.int32)
            off += n
        if cfg.pair_share > 0:  # 2i+1 reads the first whole blocks of 2i's table
            for i in range(0, cfg.num_seqs - 1, 2):
                sh = int(cfg.pair_share * min(int(ctx[i]), int(ctx[i + 1]))) // bs
                bt[i + 1, :sh] = bt[i, :sh]
        tables.append(bt.to(device))
    dgen = torch.Generator(device=device).manual_seed(seed)
    num_slots = rotations * pool_blocks * bs
    shape = (num_slots, cfg.num_kv_heads, cfg.head_dim)
    q = torch.randn(cfg.num_seqs, cfg.num_q_heads, cfg.head_dim, generator=dgen, device=device)
    k = torch.randn(shape, generator=dgen, device=device).to(cfg.dtype)
    v = torch.randn(shape, generator=dgen, device=device).to(cfg.dtype)
    if layout == "head_major":
        k = k.permute(1, 0, 2).contiguous().permute(1, 0, 2)
        v = v.permute(1, 0, 2).contiguous().permute(1, 0, 2)
    elif layout != "slot_major":
        raise ValueError(f"unknown layout {layout!r}")
    return DecodeCase(
        config=cfg,
        q=q.to(cfg.dtype),
        k_cache=k,
        v_cache=v,
        block_tables=tables,
        context_lens=ctx.to(torch.int32).to(device),
        pool_blocks=pool_blocks,
    )


@dataclass(frozen=True)
class PrefillConfig:
    name: str
    num_seqs: int
    chunk: int  # query tokens per sequence
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    dtype: torch.dtype
    prefix_max: int  # cached prefix = U{0..prefix_max} tokens, per sequence
    seed: int = 0

    @property
    def n_rep(self) -> int:
        return self.num_q_heads // self.num_kv_heads

    @property
    def scale(self) -> float:
        return self.head_dim**-0.5


PREFILL_CONFIGS: dict[str, PrefillConfig] = {
    "qwen7b-prefill": PrefillConfig("qwen7b-prefill", 8, 512, 28, 4, 128, 16, torch.bfloat16, 8192, seed=4),
}


@dataclass
class PrefillCase:
    config: PrefillConfig
    q: torch.Tensor  # [total_q, H_q, D] packed
    k_cache: torch.Tensor  # [num_slots, H_kv, D]
    v_cache: torch.Tensor
    block_tables: list[torch.Tensor]  # per rotation, int32 [B, max_blocks]
    cu_seqlens_q: torch.Tensor  # int32 [B + 1]
    q_start: torch.Tensor  # int32 [B] (cached prefix lengths)
    q_lens: list[int]
    prefixes: list[int]
    pool_blocks: int  # blocks per rotation

    @property
    def flops(self) -> int:
        """Unmasked-pair flops: 4 * H_q * D * sum(q * prefix + q (q + 1) / 2)."""
        c = self.config
        pairs = sum(n * p + n * (n + 1) // 2 for n, p in zip(self.q_lens, self.prefixes))
        return 4 * c.num_q_heads * c.head_dim * pairs

    @property
    def kv_bytes(self) -> int:
        """Distinct K+V bytes the call needs (shared prefix blocks counted once)."""
        c = self.config
        esize = torch.tensor([], dtype=c.dtype).element_size()
        blocks = len({int(x) for row, n in zip(self.block_tables[0].tolist(), self._nblocks()) for x in row[:n]})
        return blocks * c.block_size * 2 * c.num_kv_heads * c.head_dim * esize

    def _nblocks(self) -> list[int]:
        bs = self.config.block_size
        return [(p + n + bs - 1) // bs for p, n in zip(self.prefixes, self.q_lens)]


def make_prefill_case(
    config: str | PrefillConfig,
    device: torch.device | str,
    *,
    seed: int | None = None,
    rotations: int = 1,
    prefixes: list[int] | None = None,
    q_lens: list[int] | None = None,
    layout: str = "head_major",
) -> PrefillCase:
    """Seeded prefill chunks over a paged pool; ``prefixes``/``q_lens`` override the
    drawn prefix lengths / chunk sizes (pairs then share only full prefix blocks)."""
    cfg = PREFILL_CONFIGS[config] if isinstance(config, str) else config
    seed = cfg.seed if seed is None else seed
    gen = torch.Generator().manual_seed(seed)
    bs, b = cfg.block_size, cfg.num_seqs
    if prefixes is None:
        prefixes = [int(x) for x in torch.randint(0, cfg.prefix_max + 1, (b,), generator=gen)]
    q_lens = [cfg.chunk] * b if q_lens is None else list(q_lens)
    if len(prefixes) != b or len(q_lens) != b:
        raise ValueError("prefixes / q_lens must have one entry per sequence")
    # pair (2i, 2i+1) shares the full blocks of a common prefix
    shared = [min(prefixes[i], prefixes[i ^ 1] if (i ^ 1) < b else prefixes[i]) // bs for i in range(b)]
    own = [(p + n + bs - 1) // bs - shared[i] for i, (p, n) in enumerate(zip(prefixes, q_lens))]
    need = sum(shared[i] for i in range(0, b, 2)) + sum(own)
    pool_blocks = math.ceil(1.25 * need) + 1
    width = max(s + o for s, o in zip(shared, own))
    tables = []
    for r in range(rotations):
        perm = (torch.randperm(pool_blocks, generator=gen) + r * pool_blocks).tolist()
        off = 0
        rows = [None] * b
        for i in range(0, b, 2):
            pre = perm[off : off + shared[i]]
            off += shared[i]
            for j in (i, i + 1):
                if j >= b:
                    continue
                mine = perm[off : off + own[j]]
                off += own[j]
                rows[j] = pre + mine
        bt = torch.zeros(b, width, dtype=torch.int32)
        for i, row in enumerate(rows):
            bt[i, : len(row)] = torch.tensor(row, dtype=torch.int32)
        tables.append(bt.to(device))
    dgen = torch.Generator(device=device).manual_seed(seed)
    num_slots = rotations * pool_blocks * bs
    shape = (num_slots, cfg.num_kv_heads, cfg.head_dim)
    cu = [0]
    for n in q_lens:
        cu.append(cu[-1] + n)
    q = torch.randn(cu[-1], cfg.num_q_heads, cfg.head_dim, generator=dgen, device=device)
    k = torch.randn(shape, generator=dgen, device=device).to(cfg.dtype)
    v = torch.randn(shape, generator=dgen, device=device).to(cfg.dtype)
    if layout == "head_major":
        k = k.permute(1, 0, 2).contiguous().permute(1, 0, 2)
        v = v.permute(1, 0, 2).contiguous().permute(1, 0, 2)
    elif layout != "slot_major":
        raise ValueError(f"unknown layout {layout!r}")
    return PrefillCase(
        config=cfg,
        q=q.to(cfg.dtype),
        k_cache=k,
        v_cache=v,
        block_tables=tables,
        cu_seqlens_q=torch.tensor(cu, dtype=torch.int32, device=device),
        q_start=torch.tensor(prefixes, dtype=torch.int32, device=device),
        q_lens=q_lens,
        prefixes=list(prefixes),
        pool_blocks=pool_blocks,
    )
