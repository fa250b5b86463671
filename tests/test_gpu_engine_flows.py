"""Engine-style flows through the seam on the GPU, with a tiny attention-only
model (random weights, head_dim 64 so the HIP block-table kernels engage).

The flows are the ones the reference engine drives the seam with
(infrared/engine/paged_engine.py: prefill with a cached prefix :194-207,
batched decode :290-332, packed mixed prefill+decode steps :461-516,
recompute preemption :553-600): whole and chunked prefill, prefix-cache block
reuse, greedy decode, a mixed step that packs one sequence's decode with
another's prefill chunk, and eviction + recompute of a sequence whose new
blocks still hold another's K/V. At every step
the logits are compared with a full recompute of the sequence by the oracle
(contiguous causal attention over all tokens, fp32, the reference's model
math of infrared/model/layers.py:79-118 and :158-180), so paging, block
sharing, chunk boundaries and packing must all be invisible.

The block allocator below is test scaffolding, not an engine.
"""

from __future__ import annotations

import pytest
import torch

from infrared_amd import PagedKVPool, metadata, rope_paged_attention
from oracle import naive as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
HID, HQ, HKV, D, L, VOCAB, BS, THETA = 256, 8, 2, 64, 2, 97, 16, 10_000.0


class TinyModel:
    """Embedding -> L x (attention + residual) -> tied logits. Attention only: the
    seam is the part under test."""

    def __init__(self, seed: int = 0) -> None:
        g = torch.Generator().manual_seed(seed)
        self.emb = torch.randn(VOCAB, HID, generator=g) * 0.5
        self.w = [
            {
                "q": torch.randn(HID, HQ * D, generator=g) / HID**0.5,
                "k": torch.randn(HID, HKV * D, generator=g) / HID**0.5,
                "v": torch.randn(HID, HKV * D, generator=g) / HID**0.5,
                "o": torch.randn(HQ * D, HID, generator=g) / (HQ * D) ** 0.5,
            }
            for _ in range(L)
        ]
        self.gw = [{n: t.to(DEV).bfloat16() for n, t in w.items()} for w in self.w]
        self.gemb = self.emb.to(DEV).bfloat16()

    def reference_logits(self, tokens: list[int], dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """Full recompute with contiguous causal attention (CPU): [len, VOCAB] fp32."""
        n = len(tokens)
        emb = self.emb.to(dtype)
        x = emb[torch.tensor(tokens)][None]  # [1, n, HID]
        pos = torch.arange(n)[None]
        cos, sin = O.rotary_cos_sin(pos, D, THETA)
        mask = O.attention_mask([0], 0, n, n, dtype)
        for w32 in self.w:
            w = {k_: t.to(dtype) for k_, t in w32.items()}
            q = (x @ w["q"]).view(1, n, HQ, D)
            k = (x @ w["k"]).view(1, n, HKV, D)
            v = (x @ w["v"]).view(1, n, HKV, D)
            q, k = O.apply_rotary_pos_emb(q, k, cos, sin)
            a = O.masked_attention(q, O.repeat_kv(k, HQ // HKV), O.repeat_kv(v, HQ // HKV), mask, D**-0.5)
            x = x + a.reshape(1, n, HQ * D) @ w["o"]
        return (x @ emb.T)[0].float()

    def forward(self, pool: PagedKVPool, paged, tokens: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        """One step over packed tokens [1, S] at absolute positions [1, S] -> logits [S, VOCAB]."""
        s = tokens.shape[1]
        x = self.gemb[tokens]  # [1, S, HID]
        cos, sin = O.rotary_cos_sin(positions.cpu(), D, THETA)
        cos, sin = cos.to(DEV), sin.to(DEV)
        for layer, w in enumerate(self.gw):
            q = (x @ w["q"]).view(1, s, HQ, D)
            k = (x @ w["k"]).view(1, s, HKV, D)
            v = (x @ w["v"]).view(1, s, HKV, D)
            a = rope_paged_attention(q, k, v, cos, sin, paged, None, layer, D**-0.5, HQ // HKV)
            x = x + a.reshape(1, s, HQ * D) @ w["o"]
        return (x @ self.gemb.T)[0].float()


class Blocks:
    """Hands out block ids; shares a prefix's full blocks between sequences."""

    def __init__(self, num_blocks: int, seed: int) -> None:
        self.free = torch.randperm(num_blocks, generator=torch.Generator().manual_seed(seed)).tolist()

    def grow(self, table: list[int], length: int) -> None:
        while len(table) * BS < length:
            table.append(self.free.pop())

    def release(self, table: list[int]) -> None:
        """Returns a table's blocks; the next grows reuse them first (LIFO)."""
        self.free.extend(reversed(table))
        table.clear()


def _step(model, pool, seqs):
    """One packed step: each (tokens, table, num_cached) forwards its new tokens."""
    paged, _ = metadata.prefill_context(
        pool, [t for _, t, _ in seqs], [nc for _, _, nc in seqs], [len(tok) for tok, _, _ in seqs]
    )
    toks = torch.tensor([x for tok, _, _ in seqs for x in tok], device=DEV)[None]
    pos = torch.tensor([nc + i for tok, _, nc in seqs for i in range(len(tok))])[None]
    logits = model.forward(pool, paged, toks, pos)
    torch.cuda.synchronize()
    pool.check_errors()
    return logits


def _decode(model, pool, tokens, table, blocks):
    """Batched decode rows through the decode kernel: one new token each."""
    for seq_tokens, tab in zip(tokens, table):
        blocks.grow(tab, len(seq_tokens))
    num_cached = [len(t) - 1 for t in tokens]
    paged, _ = metadata.decode_context(pool, table, num_cached)
    toks = torch.tensor([t[-1] for t in tokens], device=DEV)[:, None]
    pos = torch.tensor(num_cached)[:, None]
    b = len(tokens)
    x = model.gemb[toks]  # [B, 1, HID]
    cos, sin = O.rotary_cos_sin(pos, D, THETA)
    cos, sin = cos.to(DEV), sin.to(DEV)
    for layer, w in enumerate(model.gw):
        q = (x @ w["q"]).view(b, 1, HQ, D)
        k = (x @ w["k"]).view(b, 1, HKV, D)
        v = (x @ w["v"]).view(b, 1, HKV, D)
        a = rope_paged_attention(q, k, v, cos, sin, paged, None, layer, D**-0.5, HQ // HKV)
        x = x + a.reshape(b, 1, HQ * D) @ w["o"]
    torch.cuda.synchronize()
    pool.check_errors()
    return (x @ model.gemb.T)[:, 0].float()


def _check(model, got: torch.Tensor, tokens: list[int], rows: slice) -> None:
    """The paged GPU logits are as close to the fp32 recompute as the same model
    run contiguously in bf16 is (2x that error + 0.05): paging, block sharing,
    chunking and packing add nothing beyond bf16 rounding."""
    want = model.reference_logits(tokens)[rows]
    bf16 = model.reference_logits(tokens, torch.bfloat16)[rows]
    bar = 2 * (bf16 - want).abs().max().item() + 0.05
    # the bar stays a small fraction of the logits (~0.6 of ~77 here; a causal
    # bound off by one moves them by ~13), so the check cannot go vacuous
    assert bar < 0.03 * want.abs().max().item()
    err = (got.cpu() - want).abs().max().item()
    assert err <= bar, f"max-abs {err:.4f} > {bar:.4f}"


@pytest.mark.parametrize("chunks", [[37], [16, 16, 5], [1, 20, 16]])
def test_chunked_prefill_then_greedy_decode(chunks):
    """Whole or chunked prefill, then 12 greedy decode steps: every step's logits
    match the full recompute; the greedy continuation follows the oracle's."""
    model = TinyModel(1)
    pool = PagedKVPool(L, 64, BS, HKV, D, torch.bfloat16, device=DEV, strict=True)
    blocks = Blocks(64, seed=2)
    prompt = torch.randint(0, VOCAB, (sum(chunks),), generator=torch.Generator().manual_seed(3)).tolist()
    table: list[int] = []
    done = 0
    for n in chunks:
        blocks.grow(table, done + n)
        logits = _step(model, pool, [(prompt[done : done + n], table, done)])
        _check(model, logits, prompt[: done + n], slice(done, None))
        done += n
    tokens = list(prompt)
    for _ in range(12):
        ref = model.reference_logits(tokens)[-1]
        nxt = int(ref.argmax())
        tokens.append(nxt)
        got = _decode(model, pool, [tokens], [table], blocks)
        _check(model, got, tokens, slice(-1, None))


def test_prefix_cache_block_reuse():
    """A second sequence reuses the first one's two full prefix blocks and forwards
    only its own suffix; both sequences' logits match their full recomputes."""
    model = TinyModel(4)
    pool = PagedKVPool(L, 64, BS, HKV, D, torch.bfloat16, device=DEV, strict=True)
    blocks = Blocks(64, seed=5)
    g = torch.Generator().manual_seed(6)
    shared = torch.randint(0, VOCAB, (2 * BS,), generator=g).tolist()
    a_tok = shared + torch.randint(0, VOCAB, (9,), generator=g).tolist()
    b_tok = shared + torch.randint(0, VOCAB, (21,), generator=g).tolist()
    ta: list[int] = []
    blocks.grow(ta, len(a_tok))
    _step(model, pool, [(a_tok, ta, 0)])
    tb = ta[:2]  # the two full shared blocks
    blocks.grow(tb, len(b_tok))
    logits = _step(model, pool, [(b_tok[2 * BS :], tb, 2 * BS)])
    _check(model, logits, b_tok, slice(2 * BS, None))
    # decode both, sharing blocks
    a_tok.append(3)
    b_tok.append(5)
    got = _decode(model, pool, [a_tok, b_tok], [ta, tb], blocks)
    _check(model, got[:1], a_tok, slice(-1, None))
    _check(model, got[1:], b_tok, slice(-1, None))


def test_mixed_step_packs_decode_with_prefill_chunk():
    """One packed step: sequence A decodes one token while sequence B prefills a
    40-token chunk after 20 cached tokens (the mixed step); both match."""
    model = TinyModel(7)
    pool = PagedKVPool(L, 64, BS, HKV, D, torch.bfloat16, device=DEV, strict=True)
    blocks = Blocks(64, seed=8)
    g = torch.Generator().manual_seed(9)
    a_tok = torch.randint(0, VOCAB, (30,), generator=g).tolist()
    b_tok = torch.randint(0, VOCAB, (60,), generator=g).tolist()
    ta: list[int] = []
    tb: list[int] = []
    blocks.grow(ta, 30)
    blocks.grow(tb, 20)
    _step(model, pool, [(a_tok[:29], ta, 0), (b_tok[:20], tb, 0)])
    blocks.grow(tb, 60)
    logits = _step(model, pool, [(a_tok[29:], ta, 29), (b_tok[20:], tb, 20)])
    _check(model, logits[:1], a_tok, slice(29, None))
    _check(model, logits[1:], b_tok, slice(20, None))


def test_recompute_preemption_then_resume():
    """Recompute preemption as the reference engine does it
    (infrared/engine/paged_engine.py:553-600): two sequences decode in a 7-block
    pool; when the newest needs a block and none is free it is evicted (blocks
    freed), the other decodes on and finishes, then the evicted one re-prefills
    its whole history -- prompt and generated tokens -- in chunks into blocks the
    first one left (holding its stale K/V) and decodes on. Every step's logits
    match the full recompute, so nothing of the old blocks or tables leaks."""
    model = TinyModel(10)
    pool = PagedKVPool(L, 7, BS, HKV, D, torch.bfloat16, device=DEV, strict=True)
    blocks = Blocks(7, seed=11)
    g = torch.Generator().manual_seed(12)
    a = torch.randint(0, VOCAB, (40,), generator=g).tolist()
    b = torch.randint(0, VOCAB, (30,), generator=g).tolist()
    ta: list[int] = []
    tb: list[int] = []
    blocks.grow(ta, len(a))
    blocks.grow(tb, len(b))
    logits = _step(model, pool, [(a, ta, 0), (b, tb, 0)])
    _check(model, logits[: len(a)], a, slice(0, None))
    _check(model, logits[len(a) :], b, slice(0, None))

    def greedy(tokens):
        return int(model.reference_logits(tokens)[-1].argmax())

    a.append(greedy(a))
    b.append(greedy(b))
    running = {"a": (a, ta), "b": (b, tb)}
    old_tb = None
    for _ in range(20):
        # a block for each running sequence's new token; when the pool is dry
        # the newest running sequence (b) is preempted
        for name in list(running):
            tok, tab = running[name]
            if len(tab) * BS >= len(tok):
                continue
            if not blocks.free:
                old_tb = list(tb)
                blocks.release(tb)
                del running["b"]
                if name == "b":
                    continue
            blocks.grow(tab, len(tok))
        seqs = list(running.values())
        got = _decode(model, pool, [t for t, _ in seqs], [t for _, t in seqs], blocks)
        for i, (tok, _) in enumerate(seqs):
            _check(model, got[i : i + 1], tok, slice(-1, None))
            tok.append(greedy(tok))
    assert old_tb is not None and "b" not in running, "the pool never ran dry"
    # a finishes; b recomputes the K/V of its whole history (all but the token
    # it feeds next) in chunks, into a's freed blocks, then decodes on
    blocks.release(ta)
    hist = len(b) - 1
    done = 0
    for n in (16, 20, hist - 36):
        blocks.grow(tb, done + n)
        logits = _step(model, pool, [(b[done : done + n], tb, done)])
        _check(model, logits, b[: done + n], slice(done, None))
        done += n
    assert tb != old_tb[: len(tb)]
    for _ in range(8):
        got = _decode(model, pool, [b], [tb], blocks)
        _check(model, got, b, slice(-1, None))
        b.append(greedy(b))
