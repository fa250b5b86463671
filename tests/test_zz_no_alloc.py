"""ir_paged_decode_noalloc (through the C ABI) against ir_paged_decode on the
same inputs: the same kernels on the library's own scratch array instead of a
caller workspace, so the outputs must be identical bit for bit -- on two calls
in a row, the second with a smaller input (fewer sequences, shorter
contexts), then the first shape again (the counters the calls share must be
back at zero). A shape whose partial rows exceed the array is refused before
any device work."""

from __future__ import annotations

import os
import subprocess
import sys
import textwrap

import pytest
import torch

from infrared_amd import kernels
from infrared_amd._lib import check, dtype_code, lib, ptr, stream_ptr
from infrared_amd.workloads import DecodeConfig, make_decode_case
from oracle import naive as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
IR_EWORKSPACE = -3

LONG = DecodeConfig("na-long", 8, 28, 4, 128, 16, torch.bfloat16, "uniform", 3000, 20000, seed=41)
SHORT = DecodeConfig("na-short", 3, 28, 4, 128, 16, torch.bfloat16, "uniform", 100, 3000, seed=42)


def _noalloc(case, out, err, partition=0):
    cfg = case.config
    q, kc, vc, bt = case.q, case.k_cache, case.v_cache, case.block_tables[0]
    return lib().ir_paged_decode_noalloc(
        ptr(q), q.stride(0), q.stride(1), ptr(kc), ptr(vc), kc.stride(0), kc.stride(1),
        kc.shape[0] // cfg.block_size, cfg.block_size, ptr(bt), bt.stride(0), bt.shape[1], ptr(case.context_lens),
        ptr(out), out.stride(0), out.stride(1), cfg.num_seqs, cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim,
        float(cfg.scale), dtype_code(q.dtype), partition, ptr(err), stream_ptr(q.device),
    )


def _both(case):
    cfg = case.config
    bt = case.block_tables[0]
    part = kernels.default_partition(cfg.num_seqs, cfg.num_kv_heads, bt.shape[1], cfg.block_size)
    assert kernels.decode_workspace_bytes(cfg.num_seqs, cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim,
                                          bt.shape[1], cfg.block_size, part) > 0, "shape must split"
    ref = kernels.paged_decode(case.q, case.k_cache, case.v_cache, bt, case.context_lens, cfg.block_size, cfg.scale,
                               partition_tokens=part)
    out = torch.full_like(case.q, 7.0)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    check(_noalloc(case, out, err), "ir_paged_decode_noalloc")
    torch.cuda.synchronize()
    assert err.item() == 0
    return ref, out


def test_noalloc_decode_matches_the_workspace_decode():
    long_case = make_decode_case(LONG, DEV)
    short_case = make_decode_case(SHORT, DEV)
    outs = []
    for case in (long_case, short_case, long_case):
        ref, out = _both(case)
        assert torch.equal(out, ref), f"{case.config.name}: no-alloc decode differs from ir_paged_decode"
        outs.append(out)
    out = outs[1]
    cfg = SHORT
    expect = O.decode_reference(short_case.q.cpu(), short_case.k_cache.cpu(), short_case.v_cache.cpu(),
                                short_case.block_tables[0].cpu(), short_case.context_lens.cpu(), cfg.block_size,
                                cfg.scale)
    assert (out.float().cpu() - expect).abs().max().item() <= 2e-2


def test_noalloc_decode_refuses_shapes_beyond_its_scratch():
    """1024 sequences of 32k keys split into 1024-token partitions need far more
    than the 16 MiB array: refused with IR_EWORKSPACE and a message naming the
    limit (sizes are checked before any pointer is used)."""
    rc = lib().ir_paged_decode_noalloc(
        None, 0, 0, None, None, 0, 0, 0, 16, None, 2048, 2048, None, None, 0, 0, 1024, 28, 4, 128,
        0.088, 2, 1024, None, None,
    )
    assert rc == IR_EWORKSPACE
    assert "no-alloc scratch holds" in lib().ir_last_error().decode()


_FIRST_CALL_IN_CAPTURE = textwrap.dedent("""
    import sys
    sys.path.insert(0, {root!r})
    import torch
    from infrared_amd import kernels
    from infrared_amd._lib import check, dtype_code, lib, ptr, stream_ptr
    from infrared_amd.workloads import DecodeConfig, make_decode_case

    cfg = DecodeConfig("na-capture", 8, 28, 4, 128, 16, torch.bfloat16, "uniform", 3000, 20000, seed=43)
    case = make_decode_case(cfg, "cuda")
    q, kc, vc, bt = case.q, case.k_cache, case.v_cache, case.block_tables[0]
    part = kernels.default_partition(cfg.num_seqs, cfg.num_kv_heads, bt.shape[1], cfg.block_size)
    assert kernels.decode_workspace_bytes(cfg.num_seqs, cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim,
                                          bt.shape[1], cfg.block_size, part) > 0, "shape must split"
    out = torch.full_like(q, 7.0)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    # another entry point runs eagerly first (the library's code is on the device)
    kernels.paged_decode(q, kc, vc, bt, case.context_lens, cfg.block_size, cfg.scale, partition_tokens=part)
    torch.cuda.synchronize()
    print("capturing the first no-alloc call", flush=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = lib().ir_paged_decode_noalloc(
            ptr(q), q.stride(0), q.stride(1), ptr(kc), ptr(vc), kc.stride(0), kc.stride(1),
            kc.shape[0] // cfg.block_size, cfg.block_size, ptr(bt), bt.stride(0), bt.shape[1],
            ptr(case.context_lens), ptr(out), out.stride(0), out.stride(1), cfg.num_seqs, cfg.num_q_heads,
            cfg.num_kv_heads, cfg.head_dim, float(cfg.scale), dtype_code(q.dtype), part, ptr(err),
            stream_ptr(q.device))
        check(rc, "ir_paged_decode_noalloc")
    for rep in range(3):
        if rep:
            q.normal_()  # a new query for the same graph
        graph.replay()
        ref = kernels.paged_decode(q, kc, vc, bt, case.context_lens, cfg.block_size, cfg.scale,
                                   partition_tokens=part)
        torch.cuda.synchronize()
        assert err.item() == 0
        assert torch.equal(out, ref), f"replay {{rep}}: differs from ir_paged_decode"
        print(f"replay {{rep}}: equal", flush=True)
""")


def test_noalloc_first_call_inside_graph_capture():
    """In a fresh process (nothing of the no-alloc entry point set up yet; one
    eager ir_paged_decode call before), its first call is made under
    torch.cuda.graph capture: the device-array lookup
    and the counter clear happen there (the clear is a kernel, so it is
    recorded), and every replay equals ir_paged_decode bit for bit, also after
    the query changes in place."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    res = subprocess.run([sys.executable, "-u", "-c", _FIRST_CALL_IN_CAPTURE.format(root=root)], cwd=root,
                         capture_output=True, text=True, timeout=240)
    print(res.stdout)
    assert res.returncode == 0, res.stderr[-4000:]
    assert "replay 2: equal" in res.stdout
