"""GPU parity of the chunked-prefill MFMA kernel (ir_paged_prefill, through the
C ABI) against the CPU oracle's per-sequence causal restatement
(oracle.naive.prefill_reference) on the same seeded inputs.

Bar: max-abs error <= 2e-2 for bf16/fp16 against the fp32 reference.
"""

from __future__ import annotations

import pytest
import torch

from infrared_amd import kernels
from infrared_amd._lib import ERR_BLOCK_RANGE, ERR_CONTEXT_RANGE
from infrared_amd.workloads import PrefillConfig, make_decode_case, make_prefill_case
from oracle import naive as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
TOL = 2e-2


def _run(case, err=None, bt=None):
    cfg = case.config
    bt = case.block_tables[0] if bt is None else bt
    return kernels.paged_prefill(
        case.q, case.k_cache, case.v_cache, bt, case.cu_seqlens_q, case.q_start, max(case.q_lens),
        cfg.block_size, cfg.scale, err_flags=err,
    )


def _check(case):
    cfg = case.config
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = _run(case, err)
    torch.cuda.synchronize()
    assert err.item() == 0
    ref = O.prefill_reference(
        case.q.cpu(), case.k_cache.cpu(), case.v_cache.cpu(), case.block_tables[0].cpu(),
        case.cu_seqlens_q.cpu(), case.q_start.cpu(), cfg.block_size, cfg.scale,
    )
    diff = (out.float().cpu() - ref).abs().max().item()
    assert diff <= TOL, f"{cfg.name}: max-abs {diff}"
    return out


def test_prefill_qwen7b_full_size_parity():
    """8 x 512-token chunks after prefixes up to 8192 (pairs sharing prefix blocks)."""
    case = make_prefill_case("qwen7b-prefill", DEV)
    assert max(case.prefixes) > 2048
    _check(case)


def test_prefill_ragged_chunks_and_prefixes():
    """Chunks of 1..512 tokens after prefixes that end mid-block, one empty chunk."""
    case = make_prefill_case(
        "qwen7b-prefill", DEV, prefixes=[0, 37, 512, 1000, 3, 3, 0, 5], q_lens=[1, 31, 100, 512, 0, 9, 64, 33]
    )
    _check(case)


_SWEEP = [
    # (dtype, h_q, h_kv, d, bs)
    (torch.bfloat16, 28, 4, 128, 16),
    (torch.bfloat16, 8, 8, 64, 16),
    (torch.bfloat16, 16, 2, 128, 32),
    (torch.bfloat16, 24, 2, 64, 4),  # 12 heads per KV head: two head groups of 8
    (torch.float16, 28, 4, 128, 1),
    (torch.float16, 12, 3, 64, 8),
    # block sizes that are not powers of two take the general addressing path
    # (64-bit slot offsets, a division per key instead of shifts)
    (torch.bfloat16, 28, 4, 128, 12),
    (torch.float16, 8, 2, 64, 24),
]


@pytest.mark.parametrize("dtype,h_q,h_kv,d,bs", _SWEEP)
@pytest.mark.parametrize("layout", ["head_major", "slot_major"])
def test_prefill_shape_sweep(dtype, h_q, h_kv, d, bs, layout):
    """GQA groups 1..12 (one or two head groups per workgroup), both head dims,
    block sizes 1..32, both pool layouts, ragged chunks."""
    cfg = PrefillConfig(f"pf-{h_q}-{h_kv}-{d}-{bs}", 5, 0, h_q, h_kv, d, bs, dtype, 0, seed=h_q * d + bs)
    case = make_prefill_case(cfg, DEV, prefixes=[0, 17, 64, 200, 95], q_lens=[33, 64, 1, 130, 47], layout=layout)
    _check(case)


def test_prefill_workgroup_sizes_agree():
    """Small batches run 4-wavefront workgroups (128 query columns), large ones
    8 (256; the full-size test above): a 2-sequence batch on 4, and 160 query
    heads per KV head, which 4 wavefronts cannot hold, on 8 -- both match the
    oracle."""
    small = PrefillConfig("pf-small", 2, 0, 28, 4, 128, 16, torch.bfloat16, 0, seed=21)
    _check(make_prefill_case(small, DEV, prefixes=[0, 300], q_lens=[256, 77]))
    wide = PrefillConfig("pf-wide-group", 2, 0, 160, 1, 64, 16, torch.bfloat16, 0, seed=22)
    _check(make_prefill_case(wide, DEV, prefixes=[40, 0], q_lens=[5, 3]))


def test_prefill_block_id_cache_reload():
    """Block size 1 and a 2600-token context: the workgroup's staged block ids
    (1024 at a time) are refilled mid-walk."""
    cfg = PrefillConfig("pf-bs1-long", 2, 0, 8, 2, 64, 1, torch.bfloat16, 0, seed=3)
    _check(make_prefill_case(cfg, DEV, prefixes=[2500, 1100], q_lens=[100, 40]))


def test_prefill_packed_mixed_step_matches_decode_kernel():
    """A mixed step: 6 decode rows (one-token chunks) and 2 prefill chunks packed
    in one call. The decode rows also match the decode kernel on the same pool."""
    cfg = PrefillConfig("pf-mixed", 8, 0, 28, 4, 128, 16, torch.bfloat16, 0, seed=21)
    prefixes = [700, 1500, 99, 2047, 16, 3000, 0, 256]
    q_lens = [1, 1, 1, 1, 1, 1, 256, 200]
    case = make_prefill_case(cfg, DEV, prefixes=prefixes, q_lens=q_lens)
    out = _check(case)
    rows = [0, 1, 2, 3, 4, 5]
    q_dec = case.q[rows]
    ctx = torch.tensor([p + 1 for p in prefixes[:6]], dtype=torch.int32, device=DEV)
    dec = kernels.paged_decode(q_dec, case.k_cache, case.v_cache, case.block_tables[0][:6].contiguous(), ctx, 16,
                               cfg.scale)
    torch.cuda.synchronize()
    assert (dec.float() - out[rows].float()).abs().max().item() <= TOL


def test_prefill_deterministic():
    case = make_prefill_case("qwen7b-prefill", DEV, prefixes=[0, 40, 300, 1000, 5, 5, 0, 0],
                             q_lens=[512, 100, 64, 200, 1, 2, 3, 4])
    a = _run(case)
    b = _run(case)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_prefill_flags_bad_block_ids_and_overlong_context():
    case = make_prefill_case("qwen7b-prefill", DEV, prefixes=[32, 0, 0, 0, 0, 0, 0, 0], q_lens=[16] * 8)
    bt = case.block_tables[0].clone()
    bt[0, 1] = case.pool_blocks + 7  # key 16..31 of sequence 0: outside the pool
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    _run(case, err, bt)
    torch.cuda.synchronize()
    assert err.item() & ERR_BLOCK_RANGE
    # a chunk reaching past what its table can hold
    err.zero_()
    qs = case.q_start.clone()
    qs[1] = bt.shape[1] * 16
    kernels.paged_prefill(case.q, case.k_cache, case.v_cache, case.block_tables[0], case.cu_seqlens_q, qs, 16, 16,
                          case.config.scale, err_flags=err)
    torch.cuda.synchronize()
    assert err.item() & ERR_CONTEXT_RANGE


def test_prefill_fp32_is_refused():
    case = make_decode_case("qwen0.5b-fp32", DEV, num_seqs=2)
    q = case.q.reshape(-1, case.q.shape[1], case.q.shape[2])
    cu = torch.tensor([0, 1, 2], dtype=torch.int32, device=DEV)
    qs = torch.tensor([3, 4], dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError, match="fp32"):
        kernels.paged_prefill(q, case.k_cache, case.v_cache, case.block_tables[0], cu, qs, 1, 16, 0.125)


def _host_weights(case, tq, n_qblocks):
    """Key tiles (64 keys) each (sequence, query block) item walks, -1 for items
    without query rows: the bounds the prefill kernel applies, from the host
    copy of the metadata."""
    cap = case.block_tables[0].shape[1] * case.config.block_size
    cu = case.cu_seqlens_q.cpu().tolist()
    qs = case.q_start.cpu().tolist()
    w = []
    for b in range(len(qs)):
        q_len = cu[b + 1] - cu[b]
        for tb in range(n_qblocks):
            if tb * tq >= q_len:
                w.append(-1)
                continue
            p0 = max(0, min(qs[b], cap))
            kmax = min(cap, p0 + min(q_len, (tb + 1) * tq))
            w.append((kmax + 63) // 64)
    return w


@pytest.mark.parametrize("prefixes,q_lens", [
    (None, None),  # the full 8 x 512-token workload (8-wavefront workgroups)
    ([0, 37, 512, 1000, 3, 3, 0, 5], [1, 31, 100, 512, 0, 9, 64, 33]),  # ragged, one empty chunk
    ([0, 300], [256, 77]),  # 4-wavefront workgroups
])
def test_prefill_order_is_a_heaviest_first_permutation(prefixes, q_lens):
    """The device-built order lists every item with work exactly once, heaviest
    first (non-increasing key-tile counts: the weights here are below the
    order's 2048 buckets, so the order is exact), then -1 for the items
    without query rows."""
    cfg = PrefillConfig("pf-order", 8 if prefixes is None else len(prefixes), 512, 28, 4, 128, 16,
                        torch.bfloat16, 512, seed=4)
    case = make_prefill_case(cfg, DEV, prefixes=prefixes, q_lens=q_lens)
    b, max_q = len(case.q_lens), max(case.q_lens)
    n = kernels.prefill_order_len(b, max_q, 28, 4)
    # query tokens per workgroup: 256 columns of 7 heads, or 128 when 256-column
    # workgroups would number fewer than the CUs
    four = -(-max_q // (256 // 7)) * 4 * b < 256
    tq = (128 if four else 256) // 7
    n_qblocks = -(-max_q // tq)
    assert n == b * n_qblocks
    order = kernels.prefill_order(case.cu_seqlens_q, case.q_start, case.q.shape[0], max_q,
                                  case.block_tables[0].shape[1], 16, 28, 4).cpu().tolist()
    w = _host_weights(case, tq, n_qblocks)
    busy = [i for i in range(n) if w[i] >= 0]
    assert sorted(i for i in order if i >= 0) == busy
    assert order[len(busy):] == [-1] * (n - len(busy))
    ws = [w[i] for i in order[: len(busy)]]
    assert ws == sorted(ws, reverse=True)


def test_prefill_order_changes_no_result_bit():
    """The same calls with and without the heaviest-first order: identical
    outputs and error flags (full workload, ragged chunks, a packed mixed step,
    bad block ids)."""
    cases = [
        make_prefill_case("qwen7b-prefill", DEV),
        make_prefill_case("qwen7b-prefill", DEV, prefixes=[0, 37, 512, 1000, 3, 3, 0, 5],
                          q_lens=[1, 31, 100, 512, 0, 9, 64, 33]),
        make_prefill_case(PrefillConfig("pf-mixed-o", 8, 0, 28, 4, 128, 16, torch.bfloat16, 0, seed=21), DEV,
                          prefixes=[700, 1500, 99, 2047, 16, 3000, 0, 256], q_lens=[1, 1, 1, 1, 1, 1, 256, 200]),
    ]
    for i, case in enumerate(cases):
        cfg = case.config
        bt = case.block_tables[0].clone()
        if i == 1:
            bt[3, 5] = case.pool_blocks + 3  # a bad block id inside sequence 3's keys
        b, max_q = len(case.q_lens), max(case.q_lens)
        order = kernels.prefill_order(case.cu_seqlens_q, case.q_start, case.q.shape[0], max_q, bt.shape[1],
                                      cfg.block_size, cfg.num_q_heads, cfg.num_kv_heads)
        outs, errs = [], []
        for o in (None, order):
            err = torch.zeros(1, dtype=torch.int32, device=DEV)
            outs.append(kernels.paged_prefill(case.q, case.k_cache, case.v_cache, bt, case.cu_seqlens_q,
                                              case.q_start, max_q, cfg.block_size, cfg.scale, err_flags=err,
                                              order=o))
            errs.append(err)
        torch.cuda.synchronize()
        assert torch.equal(outs[0], outs[1]), cfg.name
        assert errs[0].item() == errs[1].item() == (ERR_BLOCK_RANGE if i == 1 else 0)


def test_prefill_order_length_is_checked():
    case = make_prefill_case("qwen7b-prefill", DEV)
    cfg = case.config
    wrong = torch.full((7,), -1, dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError, match="order holds"):
        kernels.paged_prefill(case.q, case.k_cache, case.v_cache, case.block_tables[0], case.cu_seqlens_q,
                              case.q_start, cfg.chunk, cfg.block_size, cfg.scale, order=wrong)


_PP_CASES = {
    "c4": ("qwen7b-prefill", None, None),
    "ragged": ("qwen7b-prefill", [0, 37, 512, 1000, 3, 3, 0, 5], [1, 31, 100, 512, 0, 9, 64, 33]),
    # fp16, head_dim 64, a 12-token block (general addressing path), 8-wavefront workgroups
    "f16-bs12": (PrefillConfig("pf-pp-f16", 8, 0, 32, 8, 64, 12, torch.float16, 0, seed=31),
                 [0, 100, 7, 300, 12, 0, 50, 1], [300, 256, 290, 200, 310, 280, 260, 299]),
}

_PP_CHILD = r"""
import sys, torch
sys.path.insert(0, {root!r})
sys.path.insert(0, {tests!r})
from test_gpu_prefill import _PP_CASES, _run
from infrared_amd.workloads import make_prefill_case
name, prefixes, q_lens = _PP_CASES[{key!r}]
out = _run(make_prefill_case(name, "cuda", prefixes=prefixes, q_lens=q_lens))
torch.cuda.synchronize()
torch.save(out.cpu(), {path!r})
print("PINGPONG OK")
"""


@pytest.mark.parametrize("key", list(_PP_CASES))
def test_prefill_ping_pong_schedule_matches_lockstep_bit_for_bit(key, tmp_path):
    """The 8-wavefront kernel's ping-pong schedule (waves 4..7 half an
    iteration behind 0..3) does the same arithmetic in the same order as the
    lockstep schedule: identical outputs, and both within the bar of the
    oracle. The schedule knob is read once per process, so the ping-pong run
    is a child process (IR_PREFILL_PINGPONG=1) on the same seeded case."""
    import os
    import subprocess
    import sys

    name, prefixes, q_lens = _PP_CASES[key]
    tests = os.path.dirname(os.path.abspath(__file__))
    path = str(tmp_path / "pp.pt")
    res = subprocess.run(
        [sys.executable, "-c", _PP_CHILD.format(root=os.path.dirname(tests), tests=tests, key=key, path=path)],
        env={**os.environ, "IR_PREFILL_PINGPONG": "1"}, capture_output=True, text=True, timeout=110,
    )
    assert res.returncode == 0 and "PINGPONG OK" in res.stdout, res.stdout + res.stderr[-2000:]
    case = make_prefill_case(name, DEV, prefixes=prefixes, q_lens=q_lens)
    lockstep = _run(case).cpu()
    pingpong = torch.load(path, weights_only=True)
    assert torch.equal(pingpong, lockstep)
    cfg = case.config
    ref = O.prefill_reference(
        case.q.cpu(), case.k_cache.cpu(), case.v_cache.cpu(), case.block_tables[0].cpu(),
        case.cu_seqlens_q.cpu(), case.q_start.cpu(), cfg.block_size, cfg.scale,
    )
    assert (lockstep.float() - ref).abs().max().item() <= TOL


def test_prefill_flags_understated_max_q_len():
    """A chunk longer than the host's max_q_len bound has rows no workgroup
    covers: the call flags IR_ERR_CONTEXT_RANGE instead of leaving them silently
    unwritten; with the true bound the same call is clean."""
    case = make_prefill_case("qwen7b-prefill", DEV, prefixes=[0, 64, 0, 0, 0, 0, 0, 0],
                             q_lens=[300, 40, 8, 8, 8, 8, 8, 8])
    cfg = case.config
    for max_q, flagged in ((100, True), (300, False)):
        err = torch.zeros(1, dtype=torch.int32, device=DEV)
        kernels.paged_prefill(case.q, case.k_cache, case.v_cache, case.block_tables[0], case.cu_seqlens_q,
                              case.q_start, max_q, cfg.block_size, cfg.scale, err_flags=err)
        torch.cuda.synchronize()
        assert bool(err.item() & ERR_CONTEXT_RANGE) == flagged, (max_q, err.item())


def test_prefill_order_and_kernel_replay_in_a_hip_graph():
    """A step's order build and prefill captured in one hipGraph: each of three
    replays -- with eager work clearing the output and scribbling over the order
    buffer in between -- equals the eager, unordered call bit for bit."""
    case = make_prefill_case("qwen7b-prefill", DEV)
    cfg = case.config
    b, max_q = len(case.q_lens), max(case.q_lens)
    eager = _run(case)
    out = torch.empty_like(case.q)
    buf = torch.empty(kernels.prefill_order_len(b, max_q, cfg.num_q_heads, cfg.num_kv_heads), dtype=torch.int32,
                      device=DEV)

    def call():
        order = kernels.prefill_order(case.cu_seqlens_q, case.q_start, case.q.shape[0], max_q,
                                      case.block_tables[0].shape[1], cfg.block_size, cfg.num_q_heads,
                                      cfg.num_kv_heads, buf=buf)
        kernels.paged_prefill(case.q, case.k_cache, case.v_cache, case.block_tables[0], case.cu_seqlens_q,
                              case.q_start, max_q, cfg.block_size, cfg.scale, out=out, order=order)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for _ in range(3):
        out.zero_()
        buf.fill_(-7)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
