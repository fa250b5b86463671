"""GPU parity of the fused rotary-embedding + KV scatter (ir_rope_kv_scatter,
through the C ABI): bit-identical to the oracle's restatement of
apply_rotary_pos_emb followed by PagedKVPool.write on the same inputs."""

from __future__ import annotations

import pytest
import torch

from infrared_amd import PagedContext, PagedKVPool, kernels, metadata
from infrared_amd._lib import ERR_SLOT_RANGE
from infrared_amd.paged_attention import paged_attention, rope_paged_attention
from oracle import naive as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(dtype, n, hq, hkv, d, num_slots, layout, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = torch.randn(n, hq, d, generator=g, device=DEV).to(dtype)
    k = torch.randn(n, hkv, d, generator=g, device=DEV).to(dtype)
    v = torch.randn(n, hkv, d, generator=g, device=DEV).to(dtype)
    base = torch.randn(num_slots, hkv, d, generator=g, device=DEV).to(dtype)
    if layout == "head_major":
        base = base.permute(1, 0, 2).contiguous().permute(1, 0, 2)
    pos = torch.randint(0, 32768, (n,), generator=torch.Generator().manual_seed(seed))
    cos, sin = O.rotary_cos_sin(pos, d, 1_000_000.0)
    slots = torch.randperm(num_slots, generator=torch.Generator().manual_seed(seed + 1))[:n]
    return q, k, v, base, cos, sin, slots


@pytest.mark.parametrize("layout", ["head_major", "slot_major"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("hq,hkv,d", [(28, 4, 128), (14, 2, 64), (8, 8, 16), (6, 2, 80), (4, 2, 512), (0, 3, 32), (9, 1, 128)])
def test_rope_scatter_bit_exact(dtype, hq, hkv, d, layout):
    n, num_slots = 77, 300
    q, k, v, base, cos, sin, slots = _case(dtype, n, hq, hkv, d, num_slots, layout, seed=hq + d)
    kc, vc = base.clone(), (-base).clone()
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    q_out = kernels.rope_kv_scatter(q, k, v, cos.to(DEV), sin.to(DEV), kc, vc, slots.to(DEV), err_flags=err)
    torch.cuda.synchronize()
    assert err.item() == 0
    # oracle: the reference's two steps on CPU copies
    q_ref, k_ref = O.apply_rotary_pos_emb(q.cpu()[None], k.cpu()[None], cos[None], sin[None])
    kr, vr = base.cpu().clone(), (-base).cpu().clone()
    O.pool_write(kr, vr, k_ref[0], v.cpu(), slots)
    assert torch.equal(q_out.cpu(), q_ref[0])
    assert torch.equal(kc.cpu(), kr) and torch.equal(vc.cpu(), vr)


def test_rope_scatter_wide_pool_offsets():
    """A head-major pool whose head stride is 32 MiB (row offsets past 24 bits)."""
    n, hq, hkv, d, num_slots = 300, 12, 4, 128, 1 << 17
    q, k, v, _, cos, sin, _ = _case(torch.bfloat16, n, hq, hkv, d, 8, "slot_major", seed=17)
    kc = torch.zeros(hkv, num_slots, d, dtype=torch.bfloat16, device=DEV).permute(1, 0, 2)
    vc = torch.zeros(hkv, num_slots, d, dtype=torch.bfloat16, device=DEV).permute(1, 0, 2)
    slots = torch.randperm(num_slots, generator=torch.Generator().manual_seed(18))[:n]
    slots[:4] = torch.tensor([0, num_slots - 1, 1, num_slots - 2])
    q_out = kernels.rope_kv_scatter(q, k, v, cos.to(DEV), sin.to(DEV), kc, vc, slots.to(DEV))
    torch.cuda.synchronize()
    q_ref, k_ref = O.apply_rotary_pos_emb(q.cpu()[None], k.cpu()[None], cos[None], sin[None])
    assert torch.equal(q_out.cpu(), q_ref[0])
    assert torch.equal(kc[slots.to(DEV)].cpu(), k_ref[0]) and torch.equal(vc[slots.to(DEV)].cpu(), v.cpu())
    written = torch.zeros(num_slots, dtype=torch.bool)
    written[slots] = True
    assert int(kc[(~written).to(DEV)].abs().sum()) == 0 and int(vc[(~written).to(DEV)].abs().sum()) == 0


def test_rope_scatter_in_place_skip_and_flag():
    q, k, v, base, cos, sin, slots = _case(torch.bfloat16, 40, 7, 1, 128, 64, "slot_major", seed=5)
    slots = slots.clone()
    slots[3] = -1  # padding: skipped
    slots[9] = 64  # outside the pool: skipped and flagged
    kc, vc = base.clone(), base.clone()
    q_ref, k_ref = O.apply_rotary_pos_emb(q.cpu()[None], k.cpu()[None], cos[None], sin[None])
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = kernels.rope_kv_scatter(q, k, v, cos.to(DEV), sin.to(DEV), kc, vc, slots.to(DEV), q_out=q, err_flags=err)
    torch.cuda.synchronize()
    assert out.data_ptr() == q.data_ptr() and torch.equal(q.cpu(), q_ref[0])
    assert err.item() & ERR_SLOT_RANGE
    keep = [i for i in range(40) if i not in (3, 9)]
    kr, vr = base.cpu().clone(), base.cpu().clone()
    O.pool_write(kr, vr, k_ref[0][keep], v.cpu()[keep], slots[keep])
    assert torch.equal(kc.cpu(), kr) and torch.equal(vc.cpu(), vr)


def test_rope_paged_attention_equals_reference_order():
    """rope_paged_attention(pre-RoPE q/k) == apply_rotary_pos_emb then paged_attention."""
    g = torch.Generator().manual_seed(31)
    bs, h_kv, n_rep, d, b = 16, 4, 7, 128, 5
    num_cached = torch.randint(0, 500, (b,), generator=g).tolist()
    perm = torch.randperm(300, generator=g).tolist()
    tables, off = [], 0
    for nc in num_cached:
        nb = metadata.blocks_for(nc + 1, bs)
        tables.append(perm[off : off + nb])
        off += nb
    outs = []
    for fused in (False, True):
        pool = PagedKVPool(1, 300, bs, h_kv, d, torch.bfloat16, device=DEV, strict=True)
        torch.manual_seed(0)
        pool.k.normal_()
        pool.v.normal_()
        paged, mask = metadata.decode_context(pool, tables, num_cached)
        gq = torch.Generator(device=DEV).manual_seed(3)
        q = torch.randn(b, 1, h_kv * n_rep, d, generator=gq, device=DEV).to(torch.bfloat16)
        k = torch.randn(b, 1, h_kv, d, generator=gq, device=DEV).to(torch.bfloat16)
        v = torch.randn(b, 1, h_kv, d, generator=gq, device=DEV).to(torch.bfloat16)
        cos, sin = O.rotary_cos_sin(torch.tensor(num_cached)[:, None], d, 1_000_000.0)
        cos, sin = cos.to(DEV), sin.to(DEV)
        if fused:
            out = rope_paged_attention(q, k, v, cos, sin, paged, mask, 0, d**-0.5, n_rep)
        else:
            qr, kr = O.apply_rotary_pos_emb(q, k, cos, sin)
            out = paged_attention(qr, kr, v, paged, mask, 0, d**-0.5, n_rep)
        torch.cuda.synchronize()
        outs.append((out, pool.k[0].clone(), pool.v[0].clone()))
    assert torch.equal(outs[0][1], outs[1][1]) and torch.equal(outs[0][2], outs[1][2])
    assert torch.equal(outs[0][0], outs[1][0])
