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


def _oracle_step(cfg, pool_k, pool_v, batch, inputs):
    """Scatter then attend, layer by layer, on CPU copies of the pool."""
    outs = []
    for layer in range(cfg.num_layers):
        k, v = pool_k[layer], pool_v[layer]
        O.pool_write(k, v, inputs.k_new[layer].cpu(), inputs.v_new[layer].cpu(), batch.write_slots.cpu())
        dec = O.decode_reference(inputs.q_dec[layer].cpu(), k, v, batch.dec_tables.cpu(), batch.dec_ctx.cpu(),
                                 cfg.block_size, cfg.scale)
        pre = O.prefill_reference(inputs.q_pre[layer].cpu(), k, v, batch.pre_tables.cpu(), batch.cu_seqlens_q.cpu(),
                                  batch.q_start.cpu(), cfg.block_size, cfg.scale)
        outs.append((dec, pre))
    return outs


@pytest.mark.parametrize("config,planned", [(SMALL, False), (WIDE, True)])
@pytest.mark.parametrize("overlap", [False, True])
def test_mixed_step_eager_matches_oracle_and_graph_replays(overlap, config, planned):
    """Both decode schedules inside the step: the fixed partitions (12 rows) and
    the plan built once per step and captured with the layers (72 rows)."""
    cfg, pool, batch, inputs = make_mixed_case(config, DEV)
    pk = [pool.k[i].cpu().clone() for i in range(cfg.num_layers)]
    pv = [pool.v[i].cpu().clone() for i in range(cfg.num_layers)]
    step = MixedStep(pool, batch, inputs, cfg.scale, overlap=overlap)
    assert step.planned == planned
    step.eager()
    torch.cuda.synchronize()
    assert step.err.item() == 0
    ref = _oracle_step(cfg, pk, pv, batch, inputs)
    for layer in range(cfg.num_layers):
        assert torch.equal(pool.k[layer].cpu(), pk[layer]) and torch.equal(pool.v[layer].cpu(), pv[layer])
        dec, pre = ref[layer]
        assert (step.out_dec[layer].float().cpu() - dec).abs().max().item() <= 2e-2
        assert (step.out_pre[layer].float().cpu() - pre).abs().max().item() <= 2e-2
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
