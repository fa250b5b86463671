"""Pins the CPU oracle (oracle/naive.py) before it is trusted as the checker.

Each restated function is checked against something other than itself:
torch's SDPA, an fp64 loop brute force, closed forms, the reference tests'
known answers (tests/golden/reference_kats.json), and equivalences between
differently-structured algorithms (streaming, split-KV, per-sequence). The
last section plants plausible mistakes in copies of the oracle and shows the
pins reject them.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import bruteforce
from oracle import naive as O


def _causal_case(b, sq, t, h_kv, n_rep, d, seed=0):
    """q + already-repeated K/V + causal-ish additive mask (every row attends >= 1 key).

    Mirrors the reference test helper (tests/test_triton_attention.py:32-52)."""
    g = torch.Generator().manual_seed(seed)
    h = h_kv * n_rep
    q = torch.randn(b, sq, h, d, generator=g)
    k_kv = torch.randn(b, t, h_kv, d, generator=g)
    v_kv = torch.randn(b, t, h_kv, d, generator=g)
    q_pos = torch.arange(t - sq, t)[:, None]
    allowed = torch.arange(t)[None, :] <= q_pos
    mask = torch.zeros(b, 1, sq, t).masked_fill(~allowed[None, None], torch.finfo(torch.float32).min)
    return q, k_kv, v_kv, mask, allowed, d**-0.5


# ---------------------------------------------------------------- one-shot softmax


def test_masked_attention_matches_sdpa():
    """Restates tests/test_layers.py:91-101 (causal mask, MHA)."""
    q, k, v, mask, _, scale = _causal_case(2, 6, 6, 4, 1, 8)
    got = O.masked_attention(q, k, v, mask, scale)
    ref = F.scaled_dot_product_attention(
        q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), attn_mask=mask, scale=scale
    ).transpose(1, 2)
    assert torch.allclose(got, ref, atol=1e-5)


@pytest.mark.parametrize("n_rep", [1, 3, 7])
def test_masked_attention_matches_fp64_loops(n_rep):
    q, k_kv, v_kv, mask, allowed, scale = _causal_case(2, 3, 9, 2, n_rep, 8, seed=n_rep)
    got = O.masked_attention(q, O.repeat_kv(k_kv, n_rep), O.repeat_kv(v_kv, n_rep), mask, scale)
    al = allowed[None].expand(2, -1, -1).numpy()
    ref = bruteforce.attention_loops(q.numpy(), k_kv.numpy(), v_kv.numpy(), al, scale, n_rep)
    assert np.abs(got.numpy() - ref).max() < 1e-5


def test_fully_masked_row_is_uniform_average():
    """A row masked everywhere with finfo.min averages V over all keys."""
    q, k, v, mask, _, scale = _causal_case(1, 2, 5, 1, 1, 8)
    mask = torch.full_like(mask, torch.finfo(torch.float32).min)
    got = O.masked_attention(q, k, v, mask, scale)
    assert torch.allclose(got[0, 0, 0], v[0, :, 0].mean(0), atol=1e-6)


def test_repeat_kv_head_mapping(golden):
    kat = golden["repeat_kv"]
    x = torch.randn(2, 3, kat["num_kv_heads"], 4)
    out = O.repeat_kv(x, kat["n_rep"])
    for j, g in enumerate(kat["head_to_kv"]):
        assert torch.equal(out[:, :, j], x[:, :, g])


# ---------------------------------------------------------------- streaming / split


@pytest.mark.parametrize("block_n", [1, 2, 3, 4, 7, 8, 100])
def test_blockwise_matches_one_shot(block_n):
    """Restates tests/test_triton_attention.py:58-64."""
    q, k_kv, v_kv, mask, _, scale = _causal_case(2, 5, 8, 2, 2, 8)
    k, v = O.repeat_kv(k_kv, 2), O.repeat_kv(v_kv, 2)
    ref = O.blockwise_attention(q, k, v, mask, scale, block_n)
    assert torch.allclose(ref, O.masked_attention(q, k, v, mask, scale), atol=1e-5)


@pytest.mark.parametrize("part_len", [1, 2, 3, 5, 8, 16, 37, 1000])
def test_split_kv_matches_one_shot(part_len):
    """Any partition length, including ones that do not divide the key axis."""
    q, k_kv, v_kv, mask, _, scale = _causal_case(2, 3, 37, 2, 7, 16, seed=5)
    k, v = O.repeat_kv(k_kv, 7), O.repeat_kv(v_kv, 7)
    ref = O.split_kv_attention(q, k, v, mask, scale, part_len)
    assert torch.allclose(ref, O.masked_attention(q, k, v, mask, scale), atol=1e-5)


# ---------------------------------------------------------------- paged decode


def _paged_decode_case(b, h_kv, n_rep, d, bs, num_blocks, max_ctx, seed=0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    ctx = torch.randint(1, max_ctx + 1, (b,), generator=g)
    nblk = (ctx + bs - 1) // bs
    assert int(nblk.sum()) <= num_blocks, "pool too small for the drawn contexts"
    perm = torch.randperm(num_blocks, generator=g)
    tables, off = [], 0
    for n in nblk.tolist():
        tables.append(perm[off : off + n].tolist())
        off += n
    width = int(nblk.max())
    bt = torch.zeros(b, width, dtype=torch.int32)
    for i, row in enumerate(tables):
        bt[i, : len(row)] = torch.tensor(row, dtype=torch.int32)
    slots = num_blocks * bs
    k = torch.randn(slots, h_kv, d, generator=g).to(dtype)
    v = torch.randn(slots, h_kv, d, generator=g).to(dtype)
    q = torch.randn(b, h_kv * n_rep, d, generator=g).to(dtype)
    return q, k, v, bt, ctx.to(torch.int32), tables


@pytest.mark.parametrize("bs", [4, 16])
@pytest.mark.parametrize("n_rep", [1, 7])
def test_decode_reference_matches_naive_path(bs, n_rep):
    """Per-sequence decode == gather + repeat + masked softmax on the engine's metadata."""
    q, k, v, bt, ctx, tables = _paged_decode_case(5, 2, n_rep, 64, bs, 5 * 38, 150, seed=bs + n_rep)
    t_max = int(ctx.max())
    gs = O.decode_gather_slots(tables, ctx.tolist(), bs, t_max)
    mask = O.decode_mask(ctx.tolist(), t_max, torch.float32)
    naive = O.paged_attention_naive(q[:, None], k, v, gs, mask, 64**-0.5, n_rep)[:, 0]
    ref = O.decode_reference(q, k, v, bt, ctx, bs, 64**-0.5)
    assert torch.allclose(naive, ref, atol=1e-5)


def test_decode_reference_one_hot_and_constant_v():
    """Closed forms: a dominant key returns its V row; constant V returns that constant."""
    q, k, v, bt, ctx, tables = _paged_decode_case(3, 2, 4, 64, 16, 16, 40, seed=9)
    # one-hot: key 0 of every sequence aligned with q * 1000
    for i, row in enumerate(tables):
        s0 = row[0] * 16
        for g in range(2):
            k[s0, g] = q[i, g * 4] * 1000.0
    out = O.decode_reference(q, k, v, bt, ctx, 16, 64**-0.5)
    for i, row in enumerate(tables):
        assert torch.allclose(out[i, 0], v[row[0] * 16, 0], atol=1e-5)
    v_const = torch.full_like(v, 0.37)
    out = O.decode_reference(q, k, v_const, bt, ctx, 16, 64**-0.5)
    assert torch.allclose(out, torch.full_like(out, 0.37), atol=1e-6)


def _prefill_case(prefixes, q_lens, h_kv, n_rep, d, bs, seed):
    """Pool + per-sequence block tables (random distinct blocks) + packed q."""
    g = torch.Generator().manual_seed(seed)
    lengths = [p + n for p, n in zip(prefixes, q_lens)]
    need = sum((n + bs - 1) // bs for n in lengths)
    nblocks = need + 3
    perm = torch.randperm(nblocks, generator=g).tolist()
    tables, off = [], 0
    for n in lengths:
        nb = (n + bs - 1) // bs
        tables.append(perm[off : off + nb])
        off += nb
    width = max(len(t) for t in tables)
    bt = torch.tensor([t + [0] * (width - len(t)) for t in tables], dtype=torch.int32)
    k = torch.randn(nblocks * bs, h_kv, d, generator=g)
    v = torch.randn(nblocks * bs, h_kv, d, generator=g)
    cu = [0]
    for n in q_lens:
        cu.append(cu[-1] + n)
    q = torch.randn(cu[-1], h_kv * n_rep, d, generator=g)
    return q, k, v, bt, cu, tables


@pytest.mark.parametrize("bs", [4, 16])
@pytest.mark.parametrize("n_rep", [1, 7])
def test_prefill_reference_matches_engine_prefill(bs, n_rep):
    """Per-sequence chunk after a cached prefix == the engine's prefill metadata
    (gather_slots over [0, length) + attention_mask([0], num_cached, q_len, length))
    through the naive gather / repeat_kv / masked softmax path."""
    prefixes, q_lens = [0, 5, 37, 16], [9, 1, 20, 16]
    q, k, v, bt, cu, tables = _prefill_case(prefixes, q_lens, 2, n_rep, 32, bs, seed=bs + n_rep)
    ref = O.prefill_reference(q, k, v, bt, cu, prefixes, bs, 32**-0.5)
    for b, (nc, n) in enumerate(zip(prefixes, q_lens)):
        length = nc + n
        gs = torch.tensor([[O.slot(tables[b], p, bs) for p in range(length)]])
        mask = O.attention_mask([0], nc, n, length, torch.float32)
        naive = O.paged_attention_naive(q[None, cu[b] : cu[b + 1]], k, v, gs, mask, 32**-0.5, n_rep)[0]
        assert torch.allclose(naive, ref[cu[b] : cu[b + 1]], atol=1e-5)


def test_prefill_reference_matches_packed_varlen_step():
    """All sequences packed into one row (B=1) over the union of their keys with
    varlen_mask, as the mixed step builds it, == per-sequence prefill_reference."""
    prefixes, q_lens = [3, 0, 30, 12], [1, 7, 1, 5]  # decode rows are one-token chunks
    q, k, v, bt, cu, tables = _prefill_case(prefixes, q_lens, 2, 3, 16, 8, seed=4)
    ref = O.prefill_reference(q, k, v, bt, cu, prefixes, 8, 0.25)
    k_seq, k_pos, slots = [], [], []
    for b, (nc, n) in enumerate(zip(prefixes, q_lens)):
        for p in range(nc + n):
            k_seq.append(b)
            k_pos.append(p)
            slots.append(O.slot(tables[b], p, 8))
    q_seq = torch.tensor([b for b, n in enumerate(q_lens) for _ in range(n)])
    q_pos = torch.tensor([nc + i for nc, n in zip(prefixes, q_lens) for i in range(n)])
    mask = O.varlen_mask(q_seq, q_pos, torch.tensor(k_seq), torch.tensor(k_pos), torch.float32)
    naive = O.paged_attention_naive(q[None], k, v, torch.tensor([slots]), mask, 0.25, 3)[0]
    assert torch.allclose(naive, ref, atol=1e-5)


def test_prefill_reference_closed_forms():
    """The first query of a fresh sequence sees only key 0 (output = V row 0); a
    constant V returns the constant; fp64 brute force agrees on a tiny case."""
    prefixes, q_lens = [0, 4], [6, 3]
    q, k, v, bt, cu, tables = _prefill_case(prefixes, q_lens, 1, 2, 8, 4, seed=5)
    out = O.prefill_reference(q, k, v, bt, cu, prefixes, 4, 8**-0.5)
    assert torch.allclose(out[0], v[tables[0][0] * 4, 0].expand(2, -1), atol=1e-6)
    out_c = O.prefill_reference(q, k, torch.full_like(v, -1.5), bt, cu, prefixes, 4, 8**-0.5)
    assert torch.allclose(out_c, torch.full_like(out_c, -1.5), atol=1e-6)
    # brute force on sequence 1 (prefix 4, 3 queries at positions 4..6)
    keys = torch.tensor([O.slot(tables[1], p, 4) for p in range(7)])
    allowed = (torch.arange(7)[None, :] <= torch.arange(4, 7)[:, None])[None].expand(1, -1, -1).numpy()
    ref = bruteforce.attention_loops(
        q[None, cu[1] : cu[2]].numpy(), k[keys][None].numpy(), v[keys][None].numpy(), allowed, 8**-0.5, 2
    )[0]
    assert np.abs(out[cu[1] : cu[2]].numpy() - ref).max() < 1e-5


# ---------------------------------------------------------------- rotary embedding


def test_rotary_tables_and_closed_form_rotation():
    """RoPE is a rotation of each pair (x_i, x_{i+D/2}) by pos * theta^(-2i/D): checked
    in fp64 against the fp32 restatement; position 0 is the identity (exactly)."""
    d, theta = 64, 1_000_000.0
    g = torch.Generator().manual_seed(21)
    pos = torch.tensor([[0, 1, 7, 513, 4095]])
    cos, sin = O.rotary_cos_sin(pos, d, theta)
    x = torch.randn(1, 5, 3, d, generator=g)
    q_rot, k_rot = O.apply_rotary_pos_emb(x, x.flip(2), cos, sin)
    assert torch.equal(q_rot[0, 0], x[0, 0])  # cos 1, sin 0 at position 0
    half = d // 2
    inv = np.array([theta ** (-2.0 * i / d) for i in range(half)])
    xn = x.double().numpy()
    for si, p in enumerate(pos[0].tolist()):
        ang = p * inv
        c, s_ = np.cos(ang), np.sin(ang)
        x1, x2 = xn[0, si, :, :half], xn[0, si, :, half:]
        want = np.concatenate([x1 * c - x2 * s_, x2 * c + x1 * s_], axis=-1)
        assert np.abs(q_rot[0, si].double().numpy() - want).max() < 2e-4 * max(1.0, p / 512)


def test_rotary_relative_position_invariance():
    """<rope(q, m), rope(k, n)> depends only on m - n."""
    d, theta = 128, 10_000.0
    g = torch.Generator().manual_seed(22)
    q = torch.randn(1, 1, 1, d, generator=g).double()
    k = torch.randn(1, 1, 1, d, generator=g).double()

    def dot(m, n):
        cm, sm = O.rotary_cos_sin(torch.tensor([[m]]), d, theta)
        cn, sn = O.rotary_cos_sin(torch.tensor([[n]]), d, theta)
        qm, _ = O.apply_rotary_pos_emb(q, q, cm.double(), sm.double())
        kn, _ = O.apply_rotary_pos_emb(k, k, cn.double(), sn.double())
        return float((qm * kn).sum())

    assert abs(dot(10, 3) - dot(107, 100)) < 1e-3
    assert abs(dot(10, 3) - dot(3, 10)) > 1e-3  # not symmetric in general


def test_rotary_rejects_planted_sign_error(monkeypatch):
    d = 32
    pos = torch.tensor([[5]])
    cos, sin = O.rotary_cos_sin(pos, d, 1e4)
    x = torch.randn(1, 1, 1, d, generator=torch.Generator().manual_seed(23))
    good, _ = O.apply_rotary_pos_emb(x, x, cos, sin)
    with monkeypatch.context() as m:
        m.setattr(O, "rotate_half", lambda t: torch.cat((t[..., d // 2 :], -t[..., : d // 2]), dim=-1))
        bad, _ = O.apply_rotary_pos_emb(x, x, cos, sin)
    assert (bad - good).abs().max() > 1e-2


def test_naive_bf16_close_to_fp32():
    """The bf16 restatement (bf16 einsums, fp32 softmax) stays within 2e-2 of fp32."""
    q, k, v, bt, ctx, tables = _paged_decode_case(4, 2, 7, 128, 16, 64, 200, seed=3)
    t_max = int(ctx.max())
    gs = O.decode_gather_slots(tables, ctx.tolist(), 16, t_max)
    m32 = O.decode_mask(ctx.tolist(), t_max, torch.float32)
    m16 = O.decode_mask(ctx.tolist(), t_max, torch.bfloat16)
    ref = O.paged_attention_naive(q[:, None], k, v, gs, m32, 128**-0.5, 7)
    bf = O.paged_attention_naive(
        q[:, None].bfloat16(), k.bfloat16(), v.bfloat16(), gs, m16, 128**-0.5, 7
    )
    assert (bf.float() - ref).abs().max() < 2e-2


# ---------------------------------------------------------------- metadata KATs


def test_slot_arithmetic(golden):
    kat = golden["slot_arithmetic"]
    for bt, pos, want in kat["cases"]:
        assert O.slot(bt, pos, kat["block_size"]) == want


def test_decode_gather_slots_and_mask_boundaries(golden):
    kat = golden["decode_static_inputs"]
    ctx = [n + 1 for n in kat["num_cached"]]
    gs = O.decode_gather_slots(kat["block_tables"], ctx, kat["block_size"], kat["t_max"])
    for i, (bt, n) in enumerate(zip(kat["block_tables"], ctx)):
        assert gs[i, :n].tolist() == [O.slot(bt, p, kat["block_size"]) for p in range(n)]
        assert gs[i, n:].eq(0).all()
    mask = O.decode_mask(ctx, kat["t_max"], torch.float32)
    neg = torch.finfo(torch.float32).min
    for i, n in enumerate(kat["expect"]["mask_valid_len"]):
        assert (mask[i, 0, 0, :n] == 0).all() and (mask[i, 0, 0, n:] == neg).all()


def test_varlen_mask_kat(golden):
    kat = golden["varlen_mask"]
    m = O.varlen_mask(
        torch.tensor(kat["q_seq_ids"]), torch.tensor(kat["q_pos"]),
        torch.tensor(kat["k_seq_ids"]), torch.tensor(kat["k_pos"]), torch.float32,
    )
    assert (m[0, 0] == 0).tolist() == kat["allowed"]


def test_attention_mask_left_pad_and_causal():
    """Restates the contract of tests/test_layers.py:104-116: pad columns and future keys blocked."""
    m = O.attention_mask([1, 0], 0, 3, 3, torch.float32)
    allowed = (m[:, 0] == 0).tolist()
    assert allowed[0] == [[False, False, False], [False, True, False], [False, True, True]]
    assert allowed[1] == [[True, False, False], [True, True, False], [True, True, True]]


def test_buckets_kat(golden):
    for n, want in golden["default_buckets"]["cases"]:
        assert O.default_buckets(n) == tuple(want)
    with pytest.raises(ValueError):
        O.default_buckets(0)
    kat = golden["pick_bucket"]
    for b, want in kat["cases"]:
        assert O.pick_bucket(b, tuple(kat["buckets"])) == want
    with pytest.raises(ValueError, match="exceeds largest bucket"):
        O.pick_bucket(kat["rejects"][0], tuple(kat["buckets"]))


# ---------------------------------------------------------------- planted mistakes


def test_pins_reject_planted_mistakes(monkeypatch):
    """Copies of the oracle with a plausible bug each fail a pin above."""
    q, k_kv, v_kv, mask, allowed, scale = _causal_case(2, 3, 9, 2, 3, 8, seed=11)
    al = allowed[None].expand(2, -1, -1).numpy()
    ref = bruteforce.attention_loops(q.numpy(), k_kv.numpy(), v_kv.numpy(), al, scale, 3)

    def run():
        return O.masked_attention(q, O.repeat_kv(k_kv, 3), O.repeat_kv(v_kv, 3), mask, scale).numpy()

    assert np.abs(run() - ref).max() < 1e-5
    # wrong GQA mapping: head j -> kv head j % H_kv (tile instead of interleave)
    with monkeypatch.context() as m:
        m.setattr(O, "repeat_kv", lambda x, n: x.repeat(1, 1, n, 1))
        assert np.abs(run() - ref).max() > 1e-2
    # dropped scale
    with monkeypatch.context() as m:
        orig = O.masked_attention
        m.setattr(O, "masked_attention", lambda q_, k_, v_, mk, s: orig(q_, k_, v_, mk, 1.0))
        assert np.abs(run() - ref).max() > 1e-2
    # mask ignored
    with monkeypatch.context() as m:
        orig = O.masked_attention
        m.setattr(O, "masked_attention", lambda q_, k_, v_, mk, s: orig(q_, k_, v_, mk * 0, s))
        assert np.abs(run() - ref).max() > 1e-2
    # prefill causal bound off by one (keys < position instead of <=)
    pq, pk, pv, pbt, pcu, ptab = _prefill_case([5, 0], [4, 3], 1, 2, 8, 4, seed=13)
    good = O.prefill_reference(pq, pk, pv, pbt, pcu, [5, 0], 4, 8**-0.5)
    gs = torch.tensor([[O.slot(ptab[0], p, 4) for p in range(9)]])
    naive = O.paged_attention_naive(pq[None, :4], pk, pv, gs, O.attention_mask([0], 5, 4, 9, torch.float32),
                                    8**-0.5, 2)[0]
    assert torch.allclose(naive, good[:4], atol=1e-5)
    # the same path with the causal bound off by one is rejected by that pin
    bad_allowed = torch.arange(9)[None, :] < (5 + torch.arange(4))[:, None]
    bad = O.masked_attention(
        pq[None, :4], O.repeat_kv(pk[gs[0]][None], 2), O.repeat_kv(pv[gs[0]][None], 2),
        torch.zeros(1, 1, 4, 9).masked_fill(~bad_allowed[None, None], torch.finfo(torch.float32).min), 8**-0.5,
    )[0]
    assert (bad - good[:4]).abs().max() > 1e-2
    # transposed PV operand in the split-KV merge: weights by the wrong partition max
    qq, kk, vv, mm, _, sc = _causal_case(1, 2, 20, 1, 1, 8, seed=12)
    good = O.masked_attention(qq, kk, vv, mm, sc)
    with monkeypatch.context() as m:
        m.setattr(torch, "exp", lambda x: torch.pow(2.0, x))  # base-2 without the log2e fold
        bad = O.split_kv_attention(qq, kk, vv, mm, sc, 7)
    assert (bad - good).abs().max() > 1e-3
