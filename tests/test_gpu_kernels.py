"""GPU parity of the HIP kernels (called through the C ABI) against the CPU
oracle and torch library routines on the same seeded inputs.

Bars: bit-exact for the scatter, the gathers and block-table indexing;
max-abs error <= 1e-4 for fp32 and <= 2e-2 for bf16/fp16 against an fp32
reference.
"""

from __future__ import annotations

import pytest
import torch

from infrared_amd import kernels, metadata
from infrared_amd._lib import ERR_BLOCK_RANGE, ERR_CONTEXT_RANGE, ERR_GATHER_RANGE, ERR_SLOT_RANGE
from infrared_amd.workloads import DECODE_CONFIGS, DecodeConfig, make_decode_case
from oracle import naive as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def _err():
    return torch.zeros(1, dtype=torch.int32, device=DEV)


# ------------------------------------------------------------------ scatter


@pytest.mark.parametrize("head_major", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("h_kv,d", [(2, 64), (4, 128), (1, 8), (3, 4)])
def test_scatter_bit_exact_vs_index_put(dtype, h_kv, d, head_major):
    g = torch.Generator(device=DEV).manual_seed(d + h_kv)
    num_slots, n = 512, 97
    base = torch.randn(num_slots, h_kv, d, generator=g, device=DEV).to(dtype)
    if head_major:
        base = base.permute(1, 0, 2).contiguous().permute(1, 0, 2)
    kc, vc = base.clone(), (base * -1).clone()  # clone keeps the strides
    assert kc.stride() == base.stride()
    k = torch.randn(n, h_kv, d, generator=g, device=DEV).to(dtype)
    v = torch.randn(n, h_kv, d, generator=g, device=DEV).to(dtype)
    slots = torch.randperm(num_slots, device=DEV)[:n]
    err = _err()
    kernels.kv_scatter(kc, vc, k, v, slots, err)
    want_k, want_v = base.clone(), (base * -1).clone()
    want_k[slots] = k
    want_v[slots] = v
    torch.cuda.synchronize()
    assert torch.equal(kc, want_k) and torch.equal(vc, want_v)
    assert err.item() == 0
    # the CPU oracle agrees bit for bit
    ok, ov = base.cpu(), (base * -1).cpu()
    O.pool_write(ok, ov, k.cpu(), v.cpu(), slots.cpu())
    assert torch.equal(kc.cpu(), ok) and torch.equal(vc.cpu(), ov)


def test_scatter_strided_source_skip_and_flag():
    """k/v as views of a fused projection; negative slots skip; OOB slots are flagged, not written."""
    h_q, h_kv, d, n = 28, 4, 128, 64
    qkv = torch.randn(n, h_q + 2 * h_kv, d, device=DEV).bfloat16()
    k, v = qkv[:, h_q : h_q + h_kv], qkv[:, h_q + h_kv :]
    kc = torch.zeros(1024, h_kv, d, device=DEV, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    slots = torch.arange(n, device=DEV) * 7
    slots[5] = -1
    slots[9] = 1024 + 3
    err = _err()
    kernels.kv_scatter(kc, vc, k, v, slots, err)
    torch.cuda.synchronize()
    assert err.item() == ERR_SLOT_RANGE
    keep = torch.ones(n, dtype=torch.bool, device=DEV)
    keep[5] = keep[9] = False
    want = torch.zeros_like(kc)
    want[slots[keep]] = k[keep]
    assert torch.equal(kc, want)
    want_v = torch.zeros_like(vc)
    want_v[slots[keep]] = v[keep]
    assert torch.equal(vc, want_v)


def test_scatter_duplicate_identical_rows_idempotent():
    """Pad-by-repeat rows write the same row to the same slot (infrared/engine/cuda_graph.py:22-25)."""
    kc = torch.zeros(64, 2, 64, device=DEV)
    vc = torch.zeros_like(kc)
    k = torch.randn(3, 2, 64, device=DEV)
    k = torch.cat([k, k[:1], k[:1]])
    v = k * 2
    slots = torch.tensor([10, 20, 30, 10, 10], device=DEV)
    kernels.kv_scatter(kc, vc, k, v, slots)
    torch.cuda.synchronize()
    assert torch.equal(kc[10], k[0]) and torch.equal(vc[20], v[1]) and torch.equal(kc[30], k[2])


# ------------------------------------------------------------------ gathers


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gather_slots_bit_exact(dtype):
    kc = torch.randn(300, 2, 64, device=DEV).to(dtype)
    vc = torch.randn(300, 2, 64, device=DEV).to(dtype)
    gs = torch.randint(0, 300, (3, 41), device=DEV)
    ok, ov = kernels.gather_slots(kc, vc, gs)
    wk, wv = O.pool_gather(kc.cpu(), vc.cpu(), gs.cpu())
    assert torch.equal(ok.cpu(), wk) and torch.equal(ov.cpu(), wv)
    err = _err()
    gs[1, 3] = 300
    ok, _ = kernels.gather_slots(kc, vc, gs, err)
    torch.cuda.synchronize()
    assert err.item() == ERR_GATHER_RANGE and ok[1, 3].eq(0).all()


@pytest.mark.parametrize("bs", [1, 4, 8, 16, 32])
def test_block_table_gather_bit_exact(bs):
    """Block-table indexing (slot = bt[p // bs] * bs + p % bs) against the oracle's loop."""
    g = torch.Generator().manual_seed(bs)
    b, h_kv, d = 5, 2, 64
    ctx = torch.randint(1, 200, (b,), generator=g)
    nblk = (ctx + bs - 1) // bs
    num_blocks = int(nblk.sum()) + 7
    perm = torch.randperm(num_blocks, generator=g)
    tables, off = [], 0
    for n in nblk.tolist():
        tables.append(perm[off : off + n].tolist())
        off += n
    kc = torch.randn(num_blocks * bs, h_kv, d, device=DEV).bfloat16()
    vc = torch.randn_like(kc)
    bt = metadata.block_tables_tensor(tables, DEV)
    cl = ctx.to(torch.int32).to(DEV)
    t_max = int(ctx.max()) + 5
    ok, ov = kernels.paged_gather(kc, vc, bt, cl, bs, t_max)
    gs = O.decode_gather_slots(tables, ctx.tolist(), bs, t_max)
    wk, wv = O.pool_gather(kc.cpu(), vc.cpu(), gs)
    valid = torch.arange(t_max)[None, :] < ctx[:, None]
    wk[~valid] = 0
    wv[~valid] = 0
    assert torch.equal(ok.cpu(), wk) and torch.equal(ov.cpu(), wv)


# ------------------------------------------------------------------ decode


def _check_decode(case, partition_tokens=0, seqs=None):
    cfg = case.config
    bt = case.block_tables[0]
    err = _err()
    out = kernels.paged_decode(
        case.q, case.k_cache, case.v_cache, bt, case.context_lens, cfg.block_size, cfg.scale,
        partition_tokens=partition_tokens, err_flags=err,
    )
    torch.cuda.synchronize()
    assert err.item() == 0
    ref = O.decode_reference(
        case.q.cpu(), case.k_cache.cpu(), case.v_cache.cpu(), bt.cpu(), case.context_lens.cpu(),
        cfg.block_size, cfg.scale, torch.float32, seqs=seqs,
    )
    got = out.float().cpu()
    rows = list(range(cfg.num_seqs)) if seqs is None else list(seqs)
    diff = (got[rows] - ref[rows]).abs().max().item()
    assert diff <= TOL[cfg.dtype], f"{cfg.name} P={partition_tokens}: max-abs {diff}"
    return out


@pytest.mark.parametrize("layout", ["head_major", "slot_major"])
def test_decode_qwen05b_fp32_parity(layout):
    """Qwen2.5-0.5B shape, fp32: 8 seqs, 14/2 heads, D=64, ctx U[1,512]; bar 1e-4."""
    _check_decode(make_decode_case("qwen0.5b-fp32", DEV, layout=layout))


@pytest.mark.parametrize("layout", ["head_major", "slot_major"])
@pytest.mark.parametrize("partition_tokens", [0, 256, 4096])
def test_decode_qwen7b_bf16_full_size_parity(partition_tokens, layout):
    """Qwen2.5-7B shape, bf16, full batch of 64 with ctx U[512,4096]; bar 2e-2 vs fp32,
    in both pool layouts."""
    _check_decode(make_decode_case("qwen7b-bf16", DEV, layout=layout), partition_tokens)


def test_decode_skewed_long_context_split_kv():
    """Lognormal contexts up to 32k through split-KV partitions + reduce."""
    case = make_decode_case("qwen7b-skewed", DEV)
    assert int(case.context_lens.max()) > 4096
    _check_decode(case, 512)
    _check_decode(case, 0)


_SWEEP = [
    # (dtype, h_q, h_kv, d, bs, partition)
    (torch.float32, 14, 2, 64, 16, 32),
    (torch.float32, 8, 8, 128, 16, 48),
    (torch.bfloat16, 28, 4, 128, 8, 64),
    (torch.bfloat16, 16, 2, 128, 32, 96),
    (torch.bfloat16, 40, 2, 64, 16, 16),
    (torch.bfloat16, 4, 4, 64, 1, 160),
    (torch.float16, 28, 4, 128, 16, 256),
    (torch.float16, 12, 2, 64, 4, 80),
]


@pytest.mark.parametrize("dtype,h_q,h_kv,d,bs,part", _SWEEP)
def test_decode_shape_sweep(dtype, h_q, h_kv, d, bs, part):
    """GQA groups 1..20 (two head groups at 20), both head dims, block sizes 1..32
    (per-lane and block-uniform addressing), partition sizes that split mid-block,
    and context lengths on both sides of tile and block boundaries."""
    cfg = DecodeConfig(f"sweep-{h_q}-{h_kv}-{d}-{bs}", 7, h_q, h_kv, d, bs, dtype, "uniform", 300, 300, seed=h_q + bs)
    case = make_decode_case(cfg, DEV)
    # every row owns blocks for 300 tokens; use shorter lengths within them
    case.context_lens.copy_(torch.tensor([1, 15, 16, 17, 31, 33, 300], dtype=torch.int32))
    _check_decode(case, part)


# Batches mixing empty, one-token and long rows (one row spanning many
# partitions), a single 32k-token row, and a batch wider than one workgroup.
_MIX_CFG = DecodeConfig("mixed-lengths", 8, 28, 4, 128, 16, torch.bfloat16, "uniform", 5000, 5000, seed=11)


@pytest.mark.parametrize("partition_tokens", [0, 64, 4096])
def test_decode_mixed_lengths_with_empty_rows(partition_tokens):
    case = make_decode_case(_MIX_CFG, DEV)
    case.context_lens.copy_(torch.tensor([0, 1, 5000, 0, 17, 4096, 0, 2048], dtype=torch.int32))
    out = _check_decode(case, partition_tokens)
    for r in (0, 3, 6):
        assert out[r].float().abs().max().item() == 0.0


@pytest.mark.parametrize("ctx", [1, 16, 32768])
def test_decode_single_sequence(ctx):
    """One sequence: a single key, one full tile, and 32k keys (8 default
    partitions per unit, merged by the reduce launch)."""
    cfg = DecodeConfig(f"one-seq-{ctx}", 1, 28, 4, 128, 16, torch.bfloat16, "uniform", ctx, ctx, seed=ctx)
    _check_decode(make_decode_case(cfg, DEV), 0)


def test_decode_large_batch():
    cfg = DecodeConfig("batch-600", 600, 8, 2, 64, 16, torch.float16, "uniform", 1, 64, seed=5)
    _check_decode(make_decode_case(cfg, DEV), 0)


def test_decode_all_rows_empty():
    case = make_decode_case(_MIX_CFG, DEV)
    case.context_lens.zero_()
    out = _check_decode(case, 0)
    assert out.float().abs().max().item() == 0.0


_VARIANT_CHILD = r"""
import sys, torch
sys.path.insert(0, {root!r})
from infrared_amd import kernels
from infrared_amd.workloads import DecodeConfig, make_decode_case
from oracle import naive as O
for ctx, part in ((5000, 256), (777, 64), (4096, 0)):
    cfg = DecodeConfig("variant", 8, 28, 4, 128, 16, torch.bfloat16, "uniform", 1, ctx, seed=ctx)
    case = make_decode_case(cfg, "cuda")
    bt = case.block_tables[0]
    out = kernels.paged_decode(case.q, case.k_cache, case.v_cache, bt, case.context_lens, 16, cfg.scale,
                               partition_tokens=part)
    ref = O.decode_reference(case.q.cpu(), case.k_cache.cpu(), case.v_cache.cpu(), bt.cpu(),
                             case.context_lens.cpu(), 16, cfg.scale, torch.float32)
    diff = (out.float().cpu() - ref).abs().max().item()
    print(ctx, part, diff, flush=True)
    assert diff <= 2e-2, diff
print("VARIANT OK")
"""


@pytest.mark.parametrize(
    "env",
    [{"IR_DECODE_MERGE": "kernel", "IR_DECODE_DEPTH": "2"}, {"IR_DECODE_DEPTH": "3", "IR_DECODE_WAVES": "8"}],
    ids=["reduce-launch-depth2", "depth3-waves8"],
)
def test_decode_launch_variants(env):
    """The tuning knobs' other launch shapes (a second merge launch, deeper load
    rings, 8 wavefronts) keep the oracle's results on split and unsplit
    sequences. The knobs are read once per process, so each runs in a child."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    res = subprocess.run(
        [sys.executable, "-c", _VARIANT_CHILD.format(root=root)], env={**os.environ, **env},
        capture_output=True, text=True, timeout=110, cwd=root,
    )
    assert res.returncode == 0 and "VARIANT OK" in res.stdout, res.stdout + res.stderr[-2000:]


def test_decode_shared_workspace_across_different_splits():
    """The partial rows start as garbage (every int32 = 2) and are shared by calls
    whose splits and batch sizes differ, as are the arrival counters; each call
    matches the oracle, repeats bit for bit and leaves the counters at zero."""
    case = make_decode_case(_MIX_CFG, DEV)
    cfg = case.config
    bt = case.block_tables[0]
    need = kernels.decode_workspace_bytes(8, 28, 4, 128, bt.shape[1], 16, 256)
    ws = torch.full((need // 4,), 2, dtype=torch.int32, device=DEV).view(torch.uint8)
    ctr = torch.zeros(kernels.decode_num_counters(8, 28, 4), dtype=torch.int32, device=DEV)
    lens = [
        torch.tensor([5000, 5000, 5000, 5000, 5000, 5000, 5000, 5000], dtype=torch.int32),
        torch.tensor([0, 1, 5000, 0, 17, 4096, 0, 2048], dtype=torch.int32),
        torch.tensor([33, 0, 0, 0, 0, 0, 0, 4999], dtype=torch.int32),
        torch.tensor([4000, 17, 5000], dtype=torch.int32),
    ]
    for cl in lens:
        cl = cl.to(DEV)
        b = cl.shape[0]
        outs = [
            kernels.paged_decode(case.q[:b], case.k_cache, case.v_cache, bt[:b], cl, 16, cfg.scale,
                                 partition_tokens=256, workspace=ws, counters=ctr)
            for _ in range(2)
        ]
        torch.cuda.synchronize()
        assert torch.equal(outs[0], outs[1])
        assert int(ctr.abs().sum()) == 0
        ref = O.decode_reference(case.q[:b].cpu(), case.k_cache.cpu(), case.v_cache.cpu(), bt[:b].cpu(), cl.cpu(), 16,
                                 cfg.scale)
        assert (outs[0].float().cpu() - ref).abs().max().item() <= TOL[cfg.dtype]


def test_decode_flags_bad_block_ids_and_contexts():
    """Out-of-pool block ids and over-long contexts are flagged and masked, never read."""
    case = make_decode_case("qwen7b-bf16", DEV, num_seqs=4)
    bt = case.block_tables[0].clone()
    bt[1, 3] = case.pool_blocks + 100
    err = _err()
    kernels.paged_decode(case.q, case.k_cache, case.v_cache, bt, case.context_lens, 16, 0.1, err_flags=err)
    torch.cuda.synchronize()
    assert err.item() & ERR_BLOCK_RANGE
    cl = case.context_lens.clone()
    cl[0] = bt.shape[1] * 16 + 50
    err.zero_()
    kernels.paged_decode(case.q, case.k_cache, case.v_cache, case.block_tables[0], cl, 16, 0.1, err_flags=err)
    torch.cuda.synchronize()
    assert err.item() & ERR_CONTEXT_RANGE


def test_decode_one_hot_probe_returns_exact_v_row():
    """A key whose score dwarfs the rest makes the output equal its V row, which pins
    the block-table address of that key exactly."""
    case = make_decode_case("qwen7b-bf16", DEV, num_seqs=3)
    bt = case.block_tables[0]
    for i in range(3):
        n = int(case.context_lens[i])
        p = n // 2 + 3
        s = int(bt[i, p // 16]) * 16 + p % 16
        for g in range(4):
            case.k_cache[s, g] = (case.q[i, 7 * g] * 64).to(case.k_cache.dtype)
            for h in range(7 * g, 7 * g + 7):
                case.q[i, h] = case.q[i, 7 * g]
    out = kernels.paged_decode(case.q, case.k_cache, case.v_cache, bt, case.context_lens, 16, 1.0)
    torch.cuda.synchronize()
    for i in range(3):
        n = int(case.context_lens[i])
        p = n // 2 + 3
        s = int(bt[i, p // 16]) * 16 + p % 16
        for h in range(28):
            assert torch.equal(out[i, h], case.v_cache[s, h // 7]), (i, h)


# ------------------------------------------------------------------ gather_slots + mask kernel


def _masked_check(q, kc, vc, gs, mask, scale, n_rep, tol):
    out = kernels.paged_attention_masked(q, kc, vc, gs, mask, scale)
    torch.cuda.synchronize()
    ref = O.paged_attention_naive(
        q.float().cpu(), kc.float().cpu(), vc.float().cpu(), gs.cpu(), mask.float().cpu(), scale, n_rep
    )
    diff = (out.float().cpu() - ref).abs().max().item()
    assert diff <= tol, diff
    return out


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_masked_decode_form_matches_naive(dtype):
    case = make_decode_case(
        DecodeConfig("m", 6, 28, 4, 128, 16, dtype, "uniform", 1, 700, seed=4), DEV
    )
    tables = [[int(x) for x in row] for row in case.block_tables[0].cpu()]
    ctx = case.context_lens.cpu().tolist()
    t_max = max(ctx) + 9
    gs = O.decode_gather_slots(tables, ctx, 16, t_max).to(DEV)
    mask = O.decode_mask(ctx, t_max, dtype).to(DEV)
    out = _masked_check(case.q[:, None], case.k_cache, case.v_cache, gs, mask, case.config.scale, 7, TOL[dtype])
    # and the block-table decode kernel agrees with it within the same bar
    dec = kernels.paged_decode(
        case.q, case.k_cache, case.v_cache, case.block_tables[0], case.context_lens, 16, case.config.scale
    )
    torch.cuda.synchronize()
    assert (dec.float() - out[:, 0].float()).abs().max().item() <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_masked_prefix_hit_prefill_matches_naive(dtype):
    """Prefill with a cached prefix: q rows [num_cached, length), causal mask with offset
    (infrared/model/inputs.py:33-54, infrared/engine/paged_engine.py:194-207)."""
    bs, h_kv, n_rep, d = 16, 2, 7, 64
    num_cached, length = 45, 83
    nb = (length + bs - 1) // bs
    table = torch.randperm(40)[:nb].tolist()
    kc = torch.randn(40 * bs, h_kv, d, device=DEV).to(dtype)
    vc = torch.randn_like(kc)
    gs = torch.tensor([[O.slot(table, p, bs) for p in range(length)]], device=DEV)
    mask = O.attention_mask([0], num_cached, length - num_cached, length, dtype).to(DEV)
    q = torch.randn(1, length - num_cached, h_kv * n_rep, d, device=DEV).to(dtype)
    _masked_check(q, kc, vc, gs, mask, d**-0.5, n_rep, TOL[dtype])


def test_masked_packed_varlen_matches_naive():
    """The packed mixed step: B=1, all chunks' queries and all histories in one frame
    with the varlen mask (infrared/engine/paged_engine.py:461-516)."""
    bs, h_kv, n_rep, d = 16, 4, 7, 128
    dtype = torch.bfloat16
    perm = torch.randperm(200).tolist()
    seqs = [(0, 5), (40, 1), (17, 1), (0, 33)]  # (num_cached, query tokens)
    tables, off = [], 0
    for start, q in seqs:
        nb = (start + q + bs - 1) // bs
        tables.append(perm[off : off + nb])
        off += nb
    q_seq, q_pos, k_seq, k_pos, gsl = [], [], [], [], []
    for i, (start, q) in enumerate(seqs):
        for p in range(start, start + q):
            q_seq.append(i)
            q_pos.append(p)
        for p in range(start + q):
            k_seq.append(i)
            k_pos.append(p)
            gsl.append(O.slot(tables[i], p, bs))
    mask = O.varlen_mask(
        torch.tensor(q_seq), torch.tensor(q_pos), torch.tensor(k_seq), torch.tensor(k_pos), dtype
    ).to(DEV)
    kc = torch.randn(200 * bs, h_kv, d, device=DEV).to(dtype)
    vc = torch.randn_like(kc)
    gs = torch.tensor([gsl], device=DEV)
    q = torch.randn(1, len(q_seq), h_kv * n_rep, d, device=DEV).to(dtype)
    _masked_check(q, kc, vc, gs, mask, d**-0.5, n_rep, TOL[dtype])


def test_masked_fully_masked_row_is_uniform_and_bad_slot_flagged():
    kc = torch.randn(64, 1, 64, device=DEV)
    vc = torch.randn_like(kc)
    gs = torch.arange(20, device=DEV)[None]
    mask = torch.zeros(1, 1, 2, 20, device=DEV)
    mask[0, 0, 1] = torch.finfo(torch.float32).min
    q = torch.randn(1, 2, 1, 64, device=DEV)
    out = _masked_check(q, kc, vc, gs, mask, 0.125, 1, 1e-4)
    assert torch.allclose(out[0, 1, 0].cpu(), vc[:20, 0].mean(0).cpu(), atol=1e-5)
    err = _err()
    gs[0, 4] = 64
    kernels.paged_attention_masked(q, kc, vc, gs, mask, 0.125, err_flags=err)
    torch.cuda.synchronize()
    assert err.item() == ERR_GATHER_RANGE


def test_config_table_is_consistent():
    for name, cfg in DECODE_CONFIGS.items():
        assert cfg.num_q_heads % cfg.num_kv_heads == 0, name
