"""GPU parity of the fused layer steps (include/nvm_model.h) against plain
torch float32 restatements of the reference ops (tests/qwen3_reference.py):
residual add + RMSNorm (layers/layernorm.py) and per-head q/k RMSNorm + RoPE
+ k/v page store (models/qwen3.py:103-133, layers/rotary_embedding.py).

The residual sum is one rounding of an exact sum: bit-identical.  Normalised
and rotated values may differ from torch by one activation ulp where the
float32 sum of squares rounds differently (different summation order):
bounded by 2 ulps, and at least 95 % of the values identical.
"""

from __future__ import annotations

import pytest
import torch

from qwen3_reference import _rms, _rope

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
ULP = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10}


def _near(a, b, dt, what):
    a, b = a.float(), b.float()
    tol = 2 * ULP[dt] * b.abs() + 1e-6
    bad = (a - b).abs() > tol
    assert not bad.any(), f"{what}: {int(bad.sum())} values beyond 2 ulps"
    assert (a == b).float().mean().item() > 0.95, f"{what}: too few identical values"


@pytest.mark.parametrize("T,H,dt", [(37, 2048, torch.bfloat16), (5, 640, torch.float16),
                                    (1, 8192, torch.bfloat16)])
def test_residual_rms_norm(T, H, dt):
    from nano_vllm_metal_amd.fused import residual_rms_norm

    g = torch.Generator(device=DEV).manual_seed(T + H)
    h = (torch.randn(T, H, device=DEV, generator=g) * 3).to(dt)
    r = torch.randn(T, H, device=DEV, generator=g).to(dt)
    w = (1 + 0.1 * torch.randn(H, device=DEV, generator=g)).to(dt)
    h2, x = residual_rms_norm(h, r, w, 1e-6)
    assert torch.equal(h2, (h.float() + r.float()).to(dt))
    _near(x, _rms(h2, w, 1e-6), dt, "norm after residual")
    h3, x3 = residual_rms_norm(h, None, w, 1e-6)
    assert h3 is h
    _near(x3, _rms(h, w, 1e-6), dt, "norm")


@pytest.mark.parametrize("Hq,Hkv,D,dt,wide", [(32, 4, 128, torch.bfloat16, False),
                                              (8, 2, 64, torch.float16, False),
                                              (4, 4, 128, torch.bfloat16, False),
                                              (32, 4, 128, torch.bfloat16, True)])
def test_qk_norm_rope_store(Hq, Hkv, D, dt, wide):
    """wide: int64 positions, page ids and slots and float32 norm weights,
    which the wrapper converts (each converted tensor must stay alive, and
    distinct, until the call is enqueued)."""
    from nano_vllm_metal_amd.fused import qk_norm_rope_store
    from nano_vllm_metal_amd.qwen3 import RoPE

    T, P, ps, max_pos = 9, 6, 4, 300
    g = torch.Generator(device=DEV).manual_seed(Hq + D)
    qkv = torch.randn(T, (Hq + 2 * Hkv) * D, device=DEV, generator=g).to(dt)
    qn = (1 + 0.2 * torch.randn(D, device=DEV, generator=g)).to(dt)
    kn = (1 + 0.2 * torch.randn(D, device=DEV, generator=g)).to(dt)
    pos = torch.randint(0, max_pos, (T,), device=DEV, generator=g).to(torch.int32)
    rope = RoPE(D, max_pos, 1e6, DEV)
    pages = torch.randperm(P, device=DEV, generator=g)[:3].to(torch.int32)
    page_ids = pages.repeat_interleave(3)[:T].clone()
    slots = (torch.arange(T, device=DEV) % 3).to(torch.int32)
    page_ids[4] = -1  # not stored
    kp = torch.zeros(P, Hkv, ps, D, dtype=dt, device=DEV)
    vp = torch.zeros_like(kp)
    if wide:
        q, k, v = qk_norm_rope_store(qkv, Hq, Hkv, D, qn.float(), kn.float(), 1e-6, pos.long(),
                                     rope.cos, rope.sin, page_ids.long(), slots.long(), kp, vp,
                                     want_kv=True)
    else:
        q, k, v = qk_norm_rope_store(qkv, Hq, Hkv, D, qn, kn, 1e-6, pos, rope.cos, rope.sin,
                                     page_ids, slots, kp, vp, want_kv=True)
    x = qkv.view(T, Hq + 2 * Hkv, D)
    rq = _rope(_rms(x[:, :Hq], qn, 1e-6), pos.long(), 1e6)
    rk = _rope(_rms(x[:, Hq:Hq + Hkv], kn, 1e-6), pos.long(), 1e6)
    rv = x[:, Hq + Hkv:]
    _near(q, rq, dt, "q")
    _near(k, rk, dt, "k")
    assert torch.equal(v, rv.float())
    for t in range(T):
        if t == 4:
            continue
        pg, sl = int(page_ids[t]), int(slots[t])
        assert torch.equal(kp[pg, :, sl], k[t].to(dt))
        assert torch.equal(vp[pg, :, sl], rv[t])
    written = torch.zeros(P, ps, dtype=torch.bool, device=DEV)
    for t in range(T):
        if t != 4:
            written[int(page_ids[t]), int(slots[t])] = True
    assert not kp.permute(0, 2, 1, 3)[~written].any()


@pytest.mark.parametrize("T,dt,k", [(32, torch.bfloat16, 4), (300, torch.float16, 4),
                                    (32, torch.bfloat16, 8), (64, torch.float16, 8)])
def test_moe_combine_residual_norm(T, dt, k):
    """nvm_moe_forward_residual_norm: h_out is bit-identical to h + Moe(x)
    (the combine's arithmetic, then one rounding), x_out the norm of it;
    top-8 takes the kernel instance with every pair's loads at once."""
    from nano_vllm_metal_amd import Moe, QuantizedWeights, quantize
    from nano_vllm_metal_amd.fused import moe_residual_rms_norm, residual_rms_norm

    H, E, I = 512, 16, 128
    g = torch.Generator(device=DEV).manual_seed(T + k)

    def qw(*shape, std=0.05):
        wq, s, b = quantize((torch.randn(shape, generator=g, device=DEV) * std).to(dt), 64, 4)
        return QuantizedWeights(s, b, 64, 4, wq)

    moe = Moe(qw(E, H, std=0.3), qw(E, I, H), qw(E, I, H), qw(E, H, I), k, True)
    x = torch.randn(T, H, device=DEV, generator=g).to(dt)
    h = (torch.randn(T, H, device=DEV, generator=g) * 2).to(dt)
    w = (1 + 0.1 * torch.randn(H, device=DEV, generator=g)).to(dt)
    h_ref, x_ref = residual_rms_norm(h, moe(x), w, 1e-6)
    h2, x2 = moe_residual_rms_norm(moe, x, h, w, 1e-6)
    assert torch.equal(h2, h_ref)
    _near(x2, x_ref, dt, "norm of the residual")


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_embedding(dt, gs):
    """nvm_embedding against the float32 dequantisation of the gathered rows,
    bit for bit (QuantizedEmbedding.__call__, layers/embed_head.py:21-36);
    ids outside the table give zero rows."""
    import numpy as np

    from nano_vllm_metal_amd import QuantizedWeights
    from nano_vllm_metal_amd.fused import embedding
    from nano_vllm_metal_amd.linear import dequantize

    g = torch.Generator().manual_seed(gs)
    V, D = 1000, 1024
    wq = torch.randint(-2 ** 31, 2 ** 31 - 1, (V, D // 8), generator=g, dtype=torch.int64)
    wq = wq.to(torch.int32).to(DEV)
    # scales and biases over many binades, both signs
    sc = (torch.randn(V, D // gs, generator=g) * 2.0 ** torch.randint(-20, 8, (V, D // gs),
                                                                     generator=g)).to(dt).to(DEV)
    bi = (torch.randn(V, D // gs, generator=g) * 2.0 ** torch.randint(-20, 8, (V, D // gs),
                                                                     generator=g)).to(dt).to(DEV)
    table = QuantizedWeights(sc, bi, gs, 4, wq)
    tokens = torch.tensor([[0, 999, 17, 17, 500], [3, -1, 1000, 2 ** 30, 42]], dtype=torch.int32,
                          device=DEV)
    got = embedding(tokens, table, dt)
    torch.cuda.synchronize()
    assert got.shape == (2, 5, D) and got.dtype == dt
    valid = (tokens >= 0) & (tokens < V)
    ids = torch.where(valid, tokens, torch.zeros_like(tokens)).long()
    want = dequantize(wq[ids], sc[ids], bi[ids], gs, 4).to(dt)
    want = torch.where(valid[..., None], want, torch.zeros_like(want))
    g_bits = got.view(torch.int16).cpu().numpy()
    w_bits = want.view(torch.int16).cpu().numpy()
    assert np.array_equal(g_bits, w_bits)
