"""Paged attention over a paged KV cache on the GPU (libnvm_moe.so).

Mirrors ``paged_attention`` of the reference (``layers/attention.py:154-230``)
and the ops it calls, ``metal.paged_attention`` and
``metal.paged_attention_int8_decode`` (``metal/bindings.cpp:50-80``): the same
arguments, masks and output (float32, ``[B, num_heads, L, D]``).  Tensors are
torch tensors on one GPU; there is no CPU fallback.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib


def paged_attention(query: torch.Tensor, key_pages: torch.Tensor, value_pages: torch.Tensor,
                    block_table: torch.Tensor, context_lens: torch.Tensor, page_size: int,
                    key_scales: torch.Tensor | None = None,
                    value_scales: torch.Tensor | None = None, scale: float | None = None,
                    mask: str | None = None, out_dtype: torch.dtype = torch.float32
                    ) -> torch.Tensor:
    """``softmax(query . paged_key^T * scale) . paged_value``.

    ``query [B, num_heads, L, D]``; ``key_pages``/``value_pages``
    ``[P, num_kv_heads, page_size, D]`` (float32, float16, bfloat16, or int8
    with ``key_scales``/``value_scales [P, num_kv_heads, page_size, 1]``);
    ``block_table [B, max_pages]`` physical page ids (negative: no page);
    ``context_lens [B]``.  ``mask`` is None or ``"causal"`` (query row i of L
    sees key positions j <= i + context_len - L).  Returns float32
    ``[B, num_heads, L, D]`` (or, with ``out_dtype`` bf16/f16, that result
    rounded once, as the model's cast after the op).
    """
    if isinstance(mask, torch.Tensor):
        raise NotImplementedError("Paged attention only supports mask=None or causal")
    if mask is not None and mask != "causal":
        raise NotImplementedError(f"unsupported mask {mask!r}")
    lib = _lib.load()
    B, Hq, L, D = query.shape
    P, Hkv, ps, Dk = key_pages.shape
    if ps != page_size:
        raise ValueError(f"paged_attention: page tensors hold {ps} slots, page_size={page_size}")
    if Dk != D:
        raise ValueError("paged_attention: q and page tensors must have the same head dimension")
    if key_pages.shape != value_pages.shape or key_pages.dtype != value_pages.dtype:
        raise ValueError("paged_attention: key_pages and value_pages must match in shape and dtype")
    if key_pages.dtype not in _lib.KV_DTYPE_CODES:
        raise ValueError(f"paged_attention: unsupported page dtype {key_pages.dtype}")
    if Hq % Hkv != 0:
        raise ValueError("paged_attention: num_heads must be divisible by num_kv_heads")
    if block_table.dim() != 2 or context_lens.dim() != 1 or block_table.shape[0] != B \
            or context_lens.shape[0] != B:
        raise ValueError("paged_attention: block_table [B, max_pages] and context_lens [B] "
                         "must match the query batch")
    dev = _lib.require_device(query, key_pages, value_pages, block_table, context_lens,
                              key_scales, value_scales)
    factor = scale if scale is not None else 1.0 / (D ** 0.5)
    q = query.to(torch.float32).reshape(B * Hq, L, D).contiguous()
    kp = key_pages.contiguous()
    vp = value_pages.contiguous()
    bt = block_table.to(torch.int32).contiguous()
    lens = context_lens.to(torch.int32).contiguous()
    ks = vs = None
    if key_pages.dtype == torch.int8:
        if key_scales is None or value_scales is None:
            raise ValueError("paged_attention: int8 pages need key_scales and value_scales")
        ks = key_scales.to(torch.float32).reshape(P, Hkv, ps).contiguous()
        vs = value_scales.to(torch.float32).reshape(P, Hkv, ps).contiguous()
    if out_dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise ValueError(f"paged_attention: unsupported out_dtype {out_dtype}")
    out = torch.empty((B * Hq, L, D), dtype=out_dtype, device=dev)
    kv = _lib.KV_DTYPE_CODES[key_pages.dtype]
    size = ctypes.c_size_t(0)
    _lib.check(lib.nvm_paged_attention_workspace_size(B * Hq, L, D, bt.shape[1], page_size, kv,
                                                      Hkv, Hq, ctypes.byref(size)))
    ws = torch.empty(max(size.value, 1), dtype=torch.uint8, device=dev)
    _lib.check(lib.nvm_paged_attention(
        q.data_ptr(), B * Hq, L, D, kp.data_ptr(), vp.data_ptr(), P, page_size, kv,
        _lib.ptr(ks), _lib.ptr(vs), bt.data_ptr(), B, bt.shape[1], lens.data_ptr(),
        float(factor), int(mask == "causal"), Hkv, Hq, _lib.KV_DTYPE_CODES[out_dtype],
        out.data_ptr(), ws.data_ptr(),
        size.value, _lib.stream_of(dev)))
    return out.reshape(B, Hq, L, D)


def causal_attention_supports(num_heads: int, num_kv_heads: int, head_dim: int) -> bool:
    """Shapes of the causal prefill kernel: head dim 64 or 128 and 1, 2, 4, 8
    or 16 query heads per kv head."""
    r = num_heads // num_kv_heads if num_kv_heads > 0 else 0
    return head_dim in (64, 128) and num_heads % max(num_kv_heads, 1) == 0 and r in (1, 2, 4, 8, 16)


def causal_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
                     act_dtype: torch.dtype, out_dtype: torch.dtype = torch.float32
                     ) -> torch.Tensor:
    """Causal attention of an initial prefill, the float32
    ``scaled_dot_product_attention(q, k, v, scale, mask="causal")`` of
    ``models/qwen3.py:134-141``: ``q [B, L, num_heads, D]``, ``k, v
    [B, L, num_kv_heads, D]`` float32 holding ``act_dtype`` values (bf16 or
    f16, as the q/k norm and RoPE step leaves them); query i sees keys j <= i
    of its own request.  Returns ``[B, L, num_heads, D]`` of ``out_dtype``
    (float32, or that result rounded once to bf16/f16)."""
    lib = _lib.load()
    if q.dim() != 4 or k.dim() != 4 or v.shape != k.shape:
        raise ValueError("causal_attention: q [B, L, Hq, D], k and v [B, L, Hkv, D]")
    B, L, Hq, D = q.shape
    if k.shape[0] != B or k.shape[1] != L or k.shape[3] != D:
        raise ValueError("causal_attention: q, k and v must share batch, length and head dim")
    Hkv = k.shape[2]
    if Hq % Hkv:
        raise ValueError("causal_attention: num_heads must be divisible by num_kv_heads")
    if out_dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise ValueError(f"causal_attention: unsupported out_dtype {out_dtype}")
    dev = _lib.require_device(q, k, v)
    qc = q.to(torch.float32).contiguous()
    kc = k.to(torch.float32).contiguous()
    vc = v.to(torch.float32).contiguous()
    out = torch.empty((B, L, Hq, D), dtype=out_dtype, device=dev)
    _lib.check(lib.nvm_causal_attention(
        qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), B, L, Hq, Hkv, D, float(scale),
        _lib.dtype_code(act_dtype), _lib.KV_DTYPE_CODES[out_dtype], out.data_ptr(),
        _lib.stream_of(dev)))
    return out
