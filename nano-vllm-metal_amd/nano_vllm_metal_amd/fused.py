"""Fused element-wise steps of the Qwen3 layer on the GPU (include/nvm_model.h).

``residual_rms_norm`` is the residual add plus ``RMSNorm`` of the reference's
block (``models/qwen3.py:244-252``, ``layers/layernorm.py``);
``qk_norm_rope_store`` is the attention block between the projections and the
attention (``models/qwen3.py:103-133``): per-head RMSNorm of q and k, RoPE,
and the k/v store into the layer's page pool.  No CPU fallback.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib


def embedding(tokens: torch.Tensor, table, dtype: torch.dtype) -> torch.Tensor:
    """``QuantizedEmbedding.__call__`` (layers/embed_head.py:21-36): the rows of
    ``table`` (a 4-bit ``QuantizedWeights`` of shape ``[V, D/8]``) for
    ``tokens``, dequantised (``q * s + b`` in float32, rounded once to
    ``dtype``, the dtype of the table's scales); shape ``[*tokens.shape, D]``.
    Ids outside ``[0, V)`` give zero rows."""
    lib = _lib.load()
    dev = _lib.require_device(tokens, table.weight, table.scales, table.biases)
    if table.scales.dtype != dtype or table.biases.dtype != dtype:
        raise ValueError("embedding: scales and biases must have the output dtype")
    V, D8 = table.weight.shape
    D = D8 * 8
    ids = tokens.reshape(-1).to(torch.int32).contiguous()
    out = torch.empty((ids.numel(), D), dtype=dtype, device=dev)
    wq = table.weight.contiguous()
    if wq.dtype == torch.uint32:
        wq = wq.view(torch.int32)
    _lib.check(lib.nvm_embedding(ids.data_ptr(), ids.numel(), wq.data_ptr(),
                                 table.scales.contiguous().data_ptr(),
                                 table.biases.contiguous().data_ptr(), V, D, table.group_size,
                                 table.bits, _lib.dtype_code(dtype), out.data_ptr(),
                                 _lib.stream_of(dev)))
    return out.reshape(*tokens.shape, D)


def residual_rms_norm(h: torch.Tensor, r: Optional[torch.Tensor], weight: torch.Tensor,
                      eps: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """``(h + r, rms_norm(h + r) * weight)``; with ``r`` None, ``(h, rms_norm(h) * weight)``."""
    lib = _lib.load()
    dev = _lib.require_device(h, r, weight)
    H = h.shape[-1]
    h2 = h.reshape(-1, H).contiguous()
    r2 = None if r is None else r.reshape(-1, H).contiguous()
    w = weight.to(h.dtype).contiguous()
    x = torch.empty_like(h2)
    h_out = torch.empty_like(h2) if r is not None else None
    _lib.check(lib.nvm_residual_rms_norm(h2.data_ptr(), _lib.ptr(r2), w.data_ptr(), h2.shape[0],
                                         H, float(eps), _lib.dtype_code(h.dtype), _lib.ptr(h_out),
                                         x.data_ptr(), _lib.stream_of(dev)))
    out_h = h if h_out is None else h_out.reshape(h.shape)
    return out_h, x.reshape(h.shape)


def qk_norm_rope_store(qkv: torch.Tensor, num_heads: int, num_kv_heads: int, head_dim: int,
                       q_norm: torch.Tensor, k_norm: torch.Tensor, eps: float,
                       positions: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                       page_ids: torch.Tensor, slots: torch.Tensor, key_pages: torch.Tensor,
                       value_pages: torch.Tensor, want_kv: bool = False):
    """``qkv [..., (Hq + 2 Hkv) * D]`` -> float32 ``q [T, Hq, D]`` (and, with
    ``want_kv``, float32 ``k, v [T, Hkv, D]``); k and v are stored at
    ``key_pages/value_pages[page_ids[t], :, slots[t]]``."""
    lib = _lib.load()
    dev = _lib.require_device(qkv, q_norm, k_norm, positions, cos, sin, page_ids, slots,
                              key_pages, value_pages)
    D = head_dim
    x = qkv.reshape(-1, (num_heads + 2 * num_kv_heads) * D).contiguous()
    T = x.shape[0]
    if key_pages.dtype != qkv.dtype or value_pages.dtype != qkv.dtype:
        raise ValueError("qk_norm_rope_store: pages must have the activation dtype")
    # the kernel addresses page p, kv head h, slot s at ((p * Hkv + h) * ps + s) * D
    for name, pg in (("key_pages", key_pages), ("value_pages", value_pages)):
        if pg.dim() != 4 or pg.shape[1] != num_kv_heads or pg.shape[3] != D:
            raise ValueError(f"qk_norm_rope_store: {name} must be [P, {num_kv_heads}, page_size, "
                             f"{D}], got {tuple(pg.shape)}")
        if not pg.is_contiguous():
            raise ValueError(f"qk_norm_rope_store: {name} must be contiguous")
    if value_pages.shape != key_pages.shape:
        raise ValueError("qk_norm_rope_store: key and value pages differ in shape")
    if q_norm.numel() != D or k_norm.numel() != D:
        raise ValueError(f"qk_norm_rope_store: q_norm/k_norm must have {D} elements")
    if cos.shape != sin.shape or cos.dim() != 2 or cos.shape[1] != D // 2:
        raise ValueError(f"qk_norm_rope_store: cos/sin must be [max_pos, {D // 2}]")
    # Converted operands are bound to locals that live until the library call
    # has been enqueued: a temporary freed inside the argument list would hand
    # its block to the next conversion, and two arguments would alias.
    idx = []
    for name, t in (("positions", positions), ("page_ids", page_ids), ("slots", slots)):
        ti = t.reshape(-1).to(torch.int32).contiguous()
        if ti.numel() != T:
            raise ValueError(f"qk_norm_rope_store: {name} must have {T} elements, got {ti.numel()}")
        idx.append(ti)
    pos_i, page_i, slot_i = idx
    qn = q_norm.to(qkv.dtype).contiguous()
    kn = k_norm.to(qkv.dtype).contiguous()
    cos_c = cos.to(torch.float32).contiguous()
    sin_c = sin.to(torch.float32).contiguous()
    q = torch.empty((T, num_heads, D), dtype=torch.float32, device=dev)
    k = torch.empty((T, num_kv_heads, D), dtype=torch.float32, device=dev) if want_kv else None
    v = torch.empty((T, num_kv_heads, D), dtype=torch.float32, device=dev) if want_kv else None
    _lib.check(lib.nvm_qk_norm_rope_store(
        x.data_ptr(), T, num_heads, num_kv_heads, D, qn.data_ptr(), kn.data_ptr(), float(eps),
        pos_i.data_ptr(), cos_c.data_ptr(), sin_c.data_ptr(), cos_c.shape[0], page_i.data_ptr(),
        slot_i.data_ptr(), key_pages.data_ptr(), value_pages.data_ptr(), key_pages.shape[0],
        key_pages.shape[2], _lib.dtype_code(qkv.dtype), q.data_ptr(), _lib.ptr(k), _lib.ptr(v),
        _lib.stream_of(dev)))
    return q, k, v


def moe_residual_rms_norm(moe, x: torch.Tensor, h: torch.Tensor, weight: torch.Tensor,
                          eps: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """The ``Moe`` block on ``x`` with its combine fused into the residual add
    and RMSNorm that follow it: ``(h + moe(x), rms_norm(h + moe(x)) * weight)``,
    where ``moe(x)`` is bit-identical to ``moe.forward(x)``."""
    from .moe import REGIMES, Moe

    if not isinstance(moe, Moe):
        raise TypeError("moe_residual_rms_norm: a Moe block is required")
    lib = _lib.load()
    dev = _lib.require_device(x, h, weight, moe.w_router.weight, moe.w_gate.weight,
                              moe.w_up.weight, moe.w_down.weight)
    *lead, H = x.shape
    if h.shape != x.shape or weight.numel() != H:
        raise ValueError("moe_residual_rms_norm: h must have the shape of x and weight H elements")
    E, I = moe.check_operands(x.dtype, H)
    x2 = x.reshape(-1, H).contiguous()
    h2 = h.reshape(-1, H).to(x.dtype).contiguous()
    T = x2.shape[0]
    ws = moe._workspace(T, H, I, E, dev)
    (wr, sr, br), (wg, sg, bg), (wu, su, bu), (wd, sd, bd) = moe._operands()
    w = weight.to(x.dtype).contiguous()
    h_out = torch.empty_like(h2)
    x_out = torch.empty_like(x2)
    _lib.check(lib.nvm_moe_forward_residual_norm(
        x2.data_ptr(), T, H, I, E, moe.num_experts_per_tok, int(bool(moe.norm_topk_prob)),
        moe.w_gate.group_size, moe.w_gate.bits, _lib.dtype_code(x.dtype),
        wr.data_ptr(), sr.data_ptr(), br.data_ptr(), wg.data_ptr(), sg.data_ptr(), bg.data_ptr(),
        wu.data_ptr(), su.data_ptr(), bu.data_ptr(), wd.data_ptr(), sd.data_ptr(), bd.data_ptr(),
        h2.data_ptr(), w.data_ptr(), float(eps), h_out.data_ptr(), x_out.data_ptr(),
        REGIMES[moe.regime], ws.data_ptr(), ws.numel(), _lib.stream_of(dev)))
    return h_out.reshape(h.shape), x_out.reshape(x.shape)
