"""CPU oracle for paged attention — TEST INFRASTRUCTURE ONLY.

Restates, in numpy float64, what the reference's paged-attention op computes:
only ``tests/`` may import it; the product path never does and has no CPU
fallback.

Reference functions restated here (paths relative to the reference's
``src/nano_vllm_metal``):

* ``paged_attention`` — ``metal/src/paged_attention.cpp:122-296`` (the CPU
  loop of ``PagedAttention``; the GPU kernels of ``paged_attention.metal``
  compute the same function).  Query row ``n`` of ``[N = B * num_heads, L, D]``
  belongs to request ``n // num_heads`` and kv head
  ``(n % num_heads) // (num_heads // num_kv_heads)``.  Key position ``j`` of
  request ``b``, for ``j < min(context_len, max_pages * page_size)``, is slot
  ``j % page_size`` of page ``block_table[b, j // page_size]``; a negative
  page id skips the position (``:218-222``).  With ``is_causal``, row ``i``
  sees ``j <= i + context_len - L`` (``:187, 225``).  Output is
  ``sum_j softmax(scale * q.k_j) v_j``, zero for a row with no visible
  position (``:282``) and for ``context_len <= 0`` (``:180-183``).  The
  reference accumulates an online softmax in float32; this restatement
  computes the same quantity exactly (float64), which is what the tests bound
  the GPU result against.
* ``paged_attention_int8_decode`` — ``:298-410``: int8 pages with one float32
  scale per (page, kv head, slot); the key and value are ``code * scale``.

Page ids at or beyond the pool (``>= P``) are skipped here as by the HIP
kernels; the reference reads past its pool there (undefined).

Parity status (see tests/test_attention_oracle.py): pinned by closed forms
(one visible position returns its value row; identical keys return the mean
of the values), by the dense formulation the reference's own tests compare
against (``tests/test_paged_attention.py:105-188``: paged attention equals
attention over the gathered dense keys and values, empty requests are zero),
and by invariants a plausible indexing mistake breaks: permuting physical
pages with the block table, repeating kv heads into query-head groups, the
causal L-row call equal to L single-row calls over growing contexts, and the
int8 path equal to float pages holding ``code * scale``.
"""

from __future__ import annotations

import numpy as np


def paged_attention(q, key_pages, value_pages, block_table, context_lens, scale: float,
                    is_causal: bool, num_kv_heads: int, num_heads: int,
                    key_scales=None, value_scales=None) -> np.ndarray:
    """``q [N, L, D]`` -> ``out [N, L, D]`` (float64)."""
    q = np.asarray(q, np.float64)
    kp = np.asarray(key_pages, np.float64)
    vp = np.asarray(value_pages, np.float64)
    if key_scales is not None:
        kp = kp * np.asarray(key_scales, np.float64).reshape(kp.shape[:3] + (1,))
        vp = vp * np.asarray(value_scales, np.float64).reshape(vp.shape[:3] + (1,))
    bt = np.asarray(block_table, np.int64)
    lens = np.asarray(context_lens, np.int64)
    N, L, D = q.shape
    P, _, page_size, _ = kp.shape
    max_pages = bt.shape[1]
    ratio = num_heads // num_kv_heads
    out = np.zeros((N, L, D))
    for n in range(N):
        b, kvh = n // num_heads, (n % num_heads) // ratio
        ctx_len = int(lens[b])
        limit = min(ctx_len, max_pages * page_size)
        if limit <= 0:
            continue
        pos = np.arange(limit)
        pages = bt[b, pos // page_size]
        ok = (pages >= 0) & (pages < P)
        pos, pages = pos[ok], pages[ok]
        keys = kp[pages, kvh, pos % page_size]      # [J, D]
        vals = vp[pages, kvh, pos % page_size]
        for i in range(L):
            vis = pos <= i + ctx_len - L if is_causal else np.ones(len(pos), bool)
            if not vis.any():
                continue
            s = keys[vis] @ q[n, i] * scale
            p = np.exp(s - s.max())
            out[n, i] = p @ vals[vis] / p.sum()
    return out


def dense_attention(q, keys, values, scale: float, causal: bool) -> np.ndarray:
    """softmax(q k^T * scale) v over dense ``keys/values [S, D]`` for ``q [L, D]``
    (the ``scaled_dot_product_attention_grouped`` comparison of the reference's
    tests); causal rows i see positions j <= i + S - L."""
    q = np.asarray(q, np.float64)
    k = np.asarray(keys, np.float64)
    v = np.asarray(values, np.float64)
    L, S = q.shape[0], k.shape[0]
    s = q @ k.T * scale
    if causal:
        s = np.where(np.arange(S)[None, :] <= np.arange(L)[:, None] + S - L, s, -np.inf)
    s = s - s.max(axis=1, keepdims=True)
    p = np.exp(s)
    return p @ v / p.sum(axis=1, keepdims=True)


def make_pool(rng, P: int, num_kv_heads: int, page_size: int, D: int):
    """Random float64 key and value pages [P, Hkv, page_size, D]."""
    return (rng.standard_normal((P, num_kv_heads, page_size, D)),
            rng.standard_normal((P, num_kv_heads, page_size, D)))


def quantize_int8(x):
    """Per-row symmetric int8 (cache/paged.py:_quantize_page_slice): scale =
    max|x| / 127 (1 for an all-zero row), code = clip(round(x / scale))."""
    x = np.asarray(x, np.float32)
    amax = np.abs(x).max(axis=-1, keepdims=True)
    scale = np.where(amax > 0, amax / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    code = np.clip(np.round(x / scale), -127, 127).astype(np.int8)
    return code, scale[..., 0]
