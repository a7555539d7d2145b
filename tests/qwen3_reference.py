"""Plain-torch float32 reference forward of the Qwen3 model (test helper).

Recomputes the whole token sequence with dense causal attention, dequantised
weights (``w = q * scale + bias``) and ordinary float32 matmuls, rounding to
the activation dtype at the points where the reference model materialises
bf16 tensors (each projection, norm, RoPE output, attention output, SwiGLU,
expert output, residual add).  It uses none of the package's kernels; the
MoE follows layers/moe.py:37-86 (precise softmax, top-k, renormalisation).
"""

from __future__ import annotations

import torch


def _deq(w):
    from nano_vllm_metal_amd import dequantize

    return dequantize(w.weight, w.scales, w.biases, w.group_size, w.bits)


def _lin(x, w, dt):
    return (x.float() @ _deq(w).T).to(dt)


def _silu(x):
    """layers/activation.py:21-24 on act tensors: each op's result is a
    rounded act tensor, as in the reference (the stable exp(-|x|) form)."""
    sig = 1 / (1 + torch.exp(-torch.abs(x)))
    sig = torch.where(x < 0, 1 - sig, sig)
    return x * sig


def _rms(x, w, eps):
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * w.float()).to(x.dtype)


def _rope(x, pos, theta):
    D = x.shape[-1]
    half = D // 2
    inv = torch.pow(torch.tensor(float(theta)), -(torch.arange(half, dtype=torch.float32) / half))
    f = torch.outer(pos.float().cpu(), inv).to(x.device)
    cos, sin = torch.cos(f)[:, None, :], torch.sin(f)[:, None, :]
    xf = x.float()
    x1, x2 = xf[..., :half], xf[..., half:]
    return torch.cat([x1 * cos - x2 * sin, x1 * sin + x2 * cos], -1).to(x.dtype)


def _moe(x, moe, dt, margins=None):
    E = moe.w_router.weight.shape[0]
    # router logits and softmax as the oracle defines them: exact sums rounded
    # once (float64 here), then the k largest probabilities with ties to the
    # lower expert index (a stable descending sort)
    logits = (x.double() @ _deq(moe.w_router).double().T).to(dt)
    probs = torch.softmax(logits.double(), -1).to(dt)
    k = moe.num_experts_per_tok
    sc, ids = torch.sort(probs.float(), dim=-1, descending=True, stable=True)
    if margins is not None and k < E:
        # Gap between the logits of the k-th and (k+1)-th expert in units of
        # the act ulp of the larger: each logit is a rounded act value, so a
        # tiny change of the layer input moves it by at most one ulp, and a
        # gap of two ulps or less can change the chosen experts.
        lk = logits.double().gather(-1, ids[:, k - 1:k])[:, 0]
        lk1 = logits.double().gather(-1, ids[:, k:k + 1])[:, 0]
        top = torch.maximum(lk.abs(), lk1.abs()).clamp_min(2.0 ** -100)
        ulp = torch.pow(2.0, torch.floor(torch.log2(top)) - (7 if dt == torch.bfloat16 else 10))
        margins.append(((lk - lk1) / ulp).cpu())
    sc, ids = sc[:, :k], ids[:, :k]
    sc = sc.to(dt)
    if moe.norm_topk_prob:
        sc = (sc.float() / sc.float().sum(-1, keepdim=True).to(dt).float()).to(dt)
    y = torch.zeros(x.shape[0], x.shape[1], dtype=torch.float32, device=x.device)
    wg, wu, wd = _deq(moe.w_gate), _deq(moe.w_up), _deq(moe.w_down)
    for t in range(x.shape[0]):
        acc = []
        for j in range(k):
            e = int(ids[t, j])
            g = (x[t].float() @ wg[e].T).to(dt)
            u = (x[t].float() @ wu[e].T).to(dt)
            h = _silu(g) * u
            d = (h.float() @ wd[e].T).to(dt)
            acc.append((d.float() * sc[t, j].float()).to(dt))
        y[t] = torch.stack([a.float() for a in acc]).sum(0)
    assert E >= k
    return y.to(dt)


def reference_logits(model, tokens, margins=None) -> torch.Tensor:
    """``tokens [L]`` -> logits ``[L, vocab]`` (float32) of every position.

    With a list ``margins``, each MoE layer appends the per-token gap between
    the logits of its k-th and (k+1)-th expert in act ulps (near-ties, where
    a one-ulp difference in the layer input can change the chosen experts)."""
    from nano_vllm_metal_amd.moe import Moe

    c = model.config
    dt = model.dtype
    L = len(tokens)
    tok = torch.as_tensor(tokens, device=model.device)
    w = model.embed_w
    h = _deq(type(w)(w.scales[tok], w.biases[tok], w.group_size, w.bits, w.weight[tok])).to(dt)
    pos = torch.arange(L)
    Hq, Hkv, D = c.num_attention_heads, c.num_key_value_heads, c.head_dim
    causal = torch.tril(torch.ones(L, L, dtype=torch.bool, device=model.device))
    for layer in model.layers:
        x = _rms(h, layer.input_norm, c.rms_norm_eps)
        q = _lin(x, layer.wq, dt).reshape(L, Hq, D)
        k = _lin(x, layer.wk, dt).reshape(L, Hkv, D)
        v = _lin(x, layer.wv, dt).reshape(L, Hkv, D)
        q = _rope(_rms(q, layer.q_norm, c.rms_norm_eps), pos, c.rope_theta)
        k = _rope(_rms(k, layer.k_norm, c.rms_norm_eps), pos, c.rope_theta)
        kr = k.float().repeat_interleave(Hq // Hkv, dim=1)
        vr = v.float().repeat_interleave(Hq // Hkv, dim=1)
        s = torch.einsum("ihd,jhd->hij", q.float(), kr) * D ** -0.5
        s = s.masked_fill(~causal[None], float("-inf"))
        o = torch.einsum("hij,jhd->ihd", torch.softmax(s, -1), vr).to(dt).reshape(L, Hq * D)
        h = h + _lin(o, layer.wo, dt)
        x = _rms(h, layer.post_norm, c.rms_norm_eps)
        if isinstance(layer.mlp, Moe):
            h = h + _moe(x, layer.mlp, dt, margins)
        else:
            m = layer.mlp
            g, u = _lin(x, m.w_gate, dt), _lin(x, m.w_up, dt)
            h = h + _lin(_silu(g) * u, m.w_down, dt)
    h = _rms(h, model.norm, c.rms_norm_eps)
    head = model.lm_head if model.lm_head is not None else model.embed_w
    return _lin(h, head, dt).float()
