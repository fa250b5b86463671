"""The mixed engine step (decode rows + prefill chunks, every layer) on the GPU:
per layer the scatter is bit-exact against index_put on the same pool, decode
and chunk outputs match the oracle, and hipGraph replays (with and without the
two-stream overlap) equal the eager step bit for bit, replay after replay."""

from __future__ import annotations

import pytest
import torch

from infrared_amd.mixed_step import MixedConfig, MixedStep, make_mixed_case
from oracle import naive as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
SMALL = MixedConfig("mixed-small", 3, 12, 1, 300, 2, 64, 40, 28, 4, 128, 16, torch.bfloat16, seed=9)
# 72 decode rows x 4 KV heads >= one unit per CU: the decode rows take the planned schedule
WIDE = MixedConfig("mixed-wide", 2, 72, 1, 600, 1, 64, 40, 28, 4, 128, 16, torch.bfloat16, seed=10)
# fp32 (the reference's fp32 path): 72 decode rows on the plan, two 300-token
# chunks after 1,100 cached tokens on the fp32 prefill kernel's own plan
WIDE32 = MixedConfig("mixed-wide-f32", 2, 72, 1, 600, 2, 300, 1100, 28, 4, 64, 16, torch.float32, seed=11)


def _oracle_step(cfg, pool_k, pool_v, batch, inputs, compute_dtype=torch.float32):
    """Scatter then attend, layer by layer, on CPU copies of the pool."""
    outs = []
    for layer in range(cfg.num_layers):
        k, v = pool_k[layer], pool_v[layer]
        O.pool_write(k, v, inputs.k_new[layer].cpu(), inputs.v_new[layer].cpu(), batch.write_slots.cpu())
        dec = O.decode_reference(inputs.q_dec[layer].cpu(), k, v, batch.dec_tables.cpu(), batch.dec_ctx.cpu(),
                                 cfg.block_size, cfg.scale, compute_dtype=compute_dtype)
        pre = O.prefill_reference(inputs.q_pre[layer].cpu(), k, v, batch.pre_tables.cpu(), batch.cu_seqlens_q.cpu(),
                                  batch.q_start.cpu(), cfg.block_size, cfg.scale, compute_dtype=compute_dtype)
        outs.append((dec, pre))
    return outs


@pytest.mark.parametrize("config,planned", [(SMALL, False), (WIDE, True), (WIDE32, True)])
@pytest.mark.parametrize("mode", ["fused-write", "separate-write", "overlap"])
def test_mixed_step_eager_matches_oracle_and_graph_replays(mode, config, planned):
    """Both decode schedules inside the step: the fixed partitions (12 rows) and
    the plan built once per step and captured with the layers (72 rows); the
    step's K/V write inside the prefill launch (the default), as its own
    launch, and with the chunks on a second stream. In fp32 (1e-4 against an
    fp64 restatement) the prefill launch writes the rows first, then attends
    on its own plan."""
    cfg, pool, batch, inputs = make_mixed_case(config, DEV)
    f32 = cfg.dtype == torch.float32
    tol = 1e-4 if f32 else 2e-2
    pk = [pool.k[i].cpu().clone() for i in range(cfg.num_layers)]
    pv = [pool.v[i].cpu().clone() for i in range(cfg.num_layers)]
    step = MixedStep(pool, batch, inputs, cfg.scale, overlap=mode == "overlap", fused=mode == "fused-write")
    assert step.fused == (mode == "fused-write")
    assert step.planned == planned
    step.eager()
    torch.cuda.synchronize()
    assert step.err.item() == 0
    if f32:
        assert step.ordered  # the chunks' fp32 plan (1,100 cached keys)
    ref = _oracle_step(cfg, pk, pv, batch, inputs, torch.float64 if f32 else torch.float32)
    for layer in range(cfg.num_layers):
        assert torch.equal(pool.k[layer].cpu(), pk[layer]) and torch.equal(pool.v[layer].cpu(), pv[layer])
        dec, pre = ref[layer]
        assert (step.out_dec[layer].double().cpu() - dec).abs().max().item() <= tol
        assert (step.out_pre[layer].double().cpu() - pre).abs().max().item() <= tol
    eager_dec, eager_pre = step.out_dec.clone(), step.out_pre.clone()
    step.capture()
    for _ in range(3):
        step.out_dec.zero_()
        step.out_pre.zero_()
        step.replay()
        torch.cuda.synchronize()
        assert torch.equal(step.out_dec, eager_dec) and torch.equal(step.out_pre, eager_pre)
        # eager work between replays
        torch.cuda.synchronize()
    assert step.err.item() == 0


def test_mixed_step_full_shape():
    """The benchmark's mixed step at its own shape: 28 layers, 224 decode rows
    (context U{256..4096}), 4 x 256-token chunks. Every layer's scatter equals
    torch's index_put on a copy of the pool taken before the step (the whole
    layer, bit for bit); decode rows and chunks match the oracle on three
    layers (a row subset of the decode); the captured step replays bit for bit."""
    cfg, pool, batch, inputs = make_mixed_case("qwen7b-mixed", DEV)
    assert (cfg.num_layers, cfg.num_decode, cfg.num_prefill, cfg.chunk) == (28, 224, 4, 256)
    layers = (0, 13, 27)
    rows = list(range(0, cfg.num_decode, 14))  # 16 decode rows
    before_k = pool.k.clone()
    before_v = pool.v.clone()
    step = MixedStep(pool, batch, inputs, cfg.scale)
    assert step.planned
    step.eager()
    torch.cuda.synchronize()
    assert step.err.item() == 0
    slots = batch.write_slots
    for layer in range(cfg.num_layers):
        before_k[layer].index_put_((slots,), inputs.k_new[layer])
        before_v[layer].index_put_((slots,), inputs.v_new[layer])
        assert torch.equal(pool.k[layer], before_k[layer]), f"layer {layer}: K scatter differs from index_put"
        assert torch.equal(pool.v[layer], before_v[layer]), f"layer {layer}: V scatter differs from index_put"
    del before_k, before_v
    torch.cuda.empty_cache()
    for layer in layers:
        kc, vc = pool.k[layer].cpu(), pool.v[layer].cpu()
        dec = O.decode_reference(inputs.q_dec[layer].cpu(), kc, vc, batch.dec_tables.cpu(), batch.dec_ctx.cpu(),
                                 cfg.block_size, cfg.scale, seqs=rows)
        err = (step.out_dec[layer].float().cpu()[rows] - dec[rows]).abs().max().item()
        assert err <= 2e-2, f"layer {layer}: decode max-abs error {err}"
        pre = O.prefill_reference(inputs.q_pre[layer].cpu(), kc, vc, batch.pre_tables.cpu(), batch.cu_seqlens_q.cpu(),
                                  batch.q_start.cpu(), cfg.block_size, cfg.scale)
        err = (step.out_pre[layer].float().cpu() - pre).abs().max().item()
        assert err <= 2e-2, f"layer {layer}: prefill max-abs error {err}"
    eager_dec, eager_pre = step.out_dec.clone(), step.out_pre.clone()
    step.capture()
    for _ in range(2):
        step.out_dec.zero_()
        step.out_pre.zero_()
        step.replay()
        torch.cuda.synchronize()
        assert torch.equal(step.out_dec, eager_dec) and torch.equal(step.out_pre, eager_pre)
    assert step.err.item() == 0
    del step, pool, inputs
    torch.cuda.empty_cache()
