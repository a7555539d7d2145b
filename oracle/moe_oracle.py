"""CPU oracle for the Qwen3 sparse-MoE block — TEST INFRASTRUCTURE ONLY.

This module restates, in numpy, what nano-vllm-metal's MoE path computes.  It
is the checker for the HIP kernels: only ``tests/``, ``__graft_entry__.smoke``
and the ``cpu_baseline`` leg of ``bench.py`` may import it.  The product path
(``nano_vllm_metal_amd``) never imports it and has no CPU fallback.

Reference functions restated here (paths relative to the reference's
``src/nano_vllm_metal``):

* ``quantize`` — the MLX affine quantizer the reference's tests call
  (``mx.quantize`` / ``nn.quantize`` / ``to_quantized``;
  ``tests/test_quantized_matmul.py:18``, ``tests/test_moe.py:39,116``).  MLX is
  not vendored; the scale/bias choice is restated from MLX 0.29.1's published
  ``affine_quantize`` as recalled (see "parity" below).  Packing follows the
  reference's own unpack loops: element ``8*w + j`` of a row lives in bits
  ``[4j, 4j+4)`` of uint32 word ``w`` (``metal/src/quantized_matmul.cpp:131-137``,
  ``metal/src/quantized_matmul.metal:37-44,109``).
* ``dequantize`` — ``w = float(q) * float(scale) + float(bias)``
  (``quantized_matmul.cpp:135``).
* ``quantized_matmul`` — ``out[M,K] = a[M,N] . dequant(b)[K,N]^T`` accumulated
  at high precision and rounded once to the activation dtype
  (``quantized_matmul.cpp:117-145``; output dtype ``a.dtype`` at ``:76-78``).
* ``route_topk`` — ``layers/moe.py:37-49``: router logits, precise softmax,
  top-k, optional renormalisation.
* ``dispatch`` — the stable ``argsort`` of ``layers/moe.py:16-20``.
* ``grouped_expert_linear`` — ``layers/moe.py:8-34``.
* ``moe_forward`` — ``Moe.__call__``, ``layers/moe.py:69-86``, with ``silu``
  from ``layers/activation.py:21-24`` (``silu_act``: its five ops, each
  rounded to act).

Rounding specification.  Every place where the reference materialises an
activation-dtype ("act", fp16 or bf16) tensor, the oracle rounds the exact
mathematical value (computed in float64) to act with round-to-nearest-even:

* logits = rnd(sum_d x[t,d] * w[e,d])
* probs  = rnd(softmax(logits)) (softmax of the act logits, in float64)
* top-k  = the k largest probs; ties go to the lower expert index
* scores = probs[ids]; with renormalisation rnd(s_j / rnd(sum_j s_j))
* gate, up = rnd(x . W^T); h = rnd(silu_act(gate) * up) with silu_act the
  reference's stable form rounded after each of its ops; down = rnd(h . Wd^T)
* y = rnd(sum_j rnd(down_j * score_j))

Parity status (what pins each function; see tests/test_oracle.py):

* dequantize / packing: pinned by closed form (identity activations return the
  dequantised rows, the known-answer pattern of test_quantized_matmul.py:13-14)
  and by hand-packed words.
* quantize: round trip |w - dequant(quant(w))| <= |scale|/2, edge values
  exact, zero exactly representable.  The exact MLX scale choice is
  **parity unpinned** (MLX is absent; it only shapes generated inputs, both
  sides consume the same packed tensors).
* route_topk: brute-force full sort on tiny inputs, all-equal logits pick
  experts 0..k-1, one-hot logits, sum of renormalised scores.  MLX's own
  float32 ulp behaviour is **parity unpinned**.
* dispatch: ``np.argsort(kind="stable")`` closed form plus bijection,
  monotone experts, bincount and exclusive-cumsum invariants.
* grouped_expert_linear / moe_forward: per-token dense loops in float64 on
  tiny shapes; k=1 with renorm equals the expert output; identical experts
  equal one expert's output.
"""

from __future__ import annotations

import statistics

import numpy as np

ACT_DTYPES = ("float16", "bfloat16")

# --------------------------------------------------------------------------
# Activation-dtype rounding
# --------------------------------------------------------------------------

_PREC = {"float16": (11, -14), "bfloat16": (8, -126)}


def round_act(v, act: str) -> np.ndarray:
    """Round float64 values to the activation dtype (RNE), returned as float64.

    The rounding is done directly from float64 (no intermediate float32):
    on the bit pattern in the normal range, and below it by scaling to the
    target ulp, where both the scaling (a power of two) and ``rint`` (ties to
    even) are exact in float64.
    """
    v = np.asarray(v, dtype=np.float64)
    if act == "float16":
        return v.astype(np.float16).astype(np.float64)
    p, emin = _PREC[act]
    # Normal range: round-to-nearest-even on the float64 bit pattern.  The
    # 52 - (p - 1) low mantissa bits are dropped; adding half an ulp minus one
    # plus the kept lsb carries exactly when RNE rounds up (also into the
    # exponent).  Values below the smallest normal take the scaling path.
    drop = 52 - (p - 1)
    if not v.flags.c_contiguous:
        v = v.copy()
    u = v.reshape(-1).view(np.uint64)
    out = np.empty_like(v)
    ou = out.reshape(-1).view(np.uint64)
    half = np.uint64((1 << (drop - 1)) - 1)
    keep = ~np.uint64((1 << drop) - 1)
    step = 1 << 20  # chunks stay cache-resident on large weight tensors
    for i in range(0, u.size, step):
        c = u[i:i + step]
        r = c >> np.uint64(drop)
        r &= np.uint64(1)
        r += c
        r += half
        r &= keep
        ou[i:i + step] = r
    big = np.abs(out) >= 2.0 ** 128  # past the largest bfloat16: overflow
    if big.any():
        out[big] = np.copysign(np.inf, v[big])
    small = np.abs(v) < 2.0 ** emin
    if not small.any():
        return out
    nz = small & (v != 0)
    out[small & (v == 0)] = v[small & (v == 0)]
    e = np.floor(np.log2(np.abs(v[nz])))
    # guard against log2 rounding at exact powers of two
    m = np.abs(v[nz]) / np.exp2(e)
    e = np.where(m >= 2.0, e + 1, np.where(m < 1.0, e - 1, e))
    e = np.maximum(e, emin)
    ulp = np.exp2(e - (p - 1))
    out[nz] = np.rint(v[nz] / ulp) * ulp
    return out


def to_bits(v, act: str) -> np.ndarray:
    """Bit patterns (uint16) of act-representable float64 values."""
    v = np.asarray(v, dtype=np.float64)
    if act == "float16":
        return v.astype(np.float16).view(np.uint16)
    f = v.astype(np.float32)
    b = f.view(np.uint32)
    assert np.all((b & 0xFFFF) == 0), "value not representable in bfloat16"
    return (b >> 16).astype(np.uint16)


def from_bits(b, act: str) -> np.ndarray:
    """float64 values of uint16 bit patterns in the act dtype."""
    b = np.asarray(b, dtype=np.uint16)
    if act == "float16":
        return b.view(np.float16).astype(np.float64)
    return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


# --------------------------------------------------------------------------
# MLX affine int4 layout
# --------------------------------------------------------------------------


def pack_nibbles(q: np.ndarray) -> np.ndarray:
    """Pack integer codes [..., n] (0..15) into uint32 [..., n/8].

    Element ``8*w + j`` goes to bits ``[4j, 4j+4)`` of word ``w``
    (quantized_matmul.cpp:131-137).
    """
    q = np.asarray(q, dtype=np.uint32)
    assert q.shape[-1] % 8 == 0
    q = q.reshape(*q.shape[:-1], q.shape[-1] // 8, 8)
    out = np.zeros(q.shape[:-1], dtype=np.uint32)
    for j in range(8):
        out |= (q[..., j] & 0xF) << np.uint32(4 * j)
    return out


def unpack_nibbles(w: np.ndarray) -> np.ndarray:
    """Inverse of :func:`pack_nibbles`: uint32 [..., n/8] -> uint8 [..., n]."""
    w = np.asarray(w, dtype=np.uint32)
    q = np.stack([(w >> np.uint32(4 * j)) & 0xF for j in range(8)], axis=-1)
    return q.reshape(*w.shape[:-1], w.shape[-1] * 8).astype(np.uint8)


def quantize(w, group_size: int = 64, bits: int = 4, act: str = "bfloat16"):
    """MLX affine quantization of ``w[..., n]`` -> (wq u32, scales, biases).

    Restates ``mx.quantize`` (MLX 0.29.1 ``affine_quantize``, recalled): per
    group, the edge with the larger magnitude is represented exactly, the
    scale is signed so that codes stay in [0, 15], and the scale is nudged so
    that zero is exactly representable.  Scales and biases are rounded to the
    act dtype and the codes are computed against the rounded values so that
    ``dequantize`` is consistent with what the kernels read.  Returned scales
    and biases are float64 arrays of act-representable values.
    """
    assert bits == 4
    w = np.asarray(w, dtype=np.float64)
    n = w.shape[-1]
    assert n % group_size == 0
    g = w.reshape(*w.shape[:-1], n // group_size, group_size)
    n_bins = (1 << bits) - 1
    eps = 1e-7
    w_max = g.max(axis=-1).astype(np.float32).astype(np.float64)
    w_min = g.min(axis=-1).astype(np.float32).astype(np.float64)
    mask = np.abs(w_min) > np.abs(w_max)
    scales = np.maximum((w_max - w_min) / n_bins, eps)
    scales = np.where(mask, scales, -scales)
    edge = np.where(mask, w_min, w_max)
    q0 = np.rint(edge / scales)
    scales = np.where(q0 != 0, edge / np.where(q0 != 0, q0, 1.0), scales)
    biases = np.where(q0 == 0, 0.0, edge)
    scales = round_act(scales, act)
    biases = round_act(biases, act)
    # a group whose scale rounds to zero would make every code meaningless
    scales = np.where(scales == 0, round_act(np.full_like(scales, eps), act), scales)
    q = np.rint((g - biases[..., None]) / scales[..., None])
    q = np.clip(q, 0, n_bins).astype(np.uint32)
    wq = pack_nibbles(q.reshape(w.shape))
    return wq, scales, biases


def dequantize(wq, scales, biases, group_size: int) -> np.ndarray:
    """``w = q * scale + bias`` in float64 (exact: q*s and the sum fit)."""
    q = unpack_nibbles(wq).astype(np.float64)
    n = q.shape[-1]
    qg = q.reshape(*q.shape[:-1], n // group_size, group_size)
    w = qg * np.asarray(scales, np.float64)[..., None] + np.asarray(biases, np.float64)[..., None]
    return w.reshape(q.shape)


# --------------------------------------------------------------------------
# The MoE path
# --------------------------------------------------------------------------


def quantized_matmul(a, wq, scales, biases, group_size: int, act: str) -> np.ndarray:
    """out = rnd(a . dequant(wq)^T) — quantized_matmul.cpp:117-145."""
    w = dequantize(wq, scales, biases, group_size)
    return round_act(np.asarray(a, np.float64) @ w.T, act)


def softmax_act(logits, act: str) -> np.ndarray:
    """rnd(softmax(logits)) along the last axis (moe.py:44, precise=True)."""
    lg = np.asarray(logits, np.float64)
    m = lg.max(axis=-1, keepdims=True)
    p = np.exp(lg - m)
    return round_act(p / p.sum(axis=-1, keepdims=True), act)


def topk_lower_index(probs, k: int) -> np.ndarray:
    """ids of the k largest probs per row, ties -> lower index, in
    (prob desc, index asc) slot order.  Replaces ``argpartition(-p)[..., :k]``
    (moe.py:45), whose slot order MLX leaves unspecified."""
    p = np.asarray(probs, np.float64)
    # stable sort of -p keeps lower indices first among equal probabilities
    order = np.argsort(-p, axis=-1, kind="stable")
    return order[..., :k].astype(np.int32)


def route_topk(x, wr, sr, br, group_size: int, top_k: int, norm_topk_prob: bool, act: str):
    """moe.py:37-49 -> (logits, probs, ids, scores), all act values as float64."""
    x2 = np.asarray(x, np.float64).reshape(-1, np.shape(x)[-1])
    logits = quantized_matmul(x2, wr, sr, br, group_size, act)
    probs = softmax_act(logits, act)
    ids = topk_lower_index(probs, top_k)
    scores = np.take_along_axis(probs, ids, axis=-1)
    if norm_topk_prob:
        denom = round_act(scores.sum(axis=-1, keepdims=True), act)
        scores = round_act(scores / denom, act)
    return logits, probs, ids, scores


def dispatch(ids, num_experts: int):
    """Stable argsort of the flat expert ids (moe.py:16-17).

    Returns ``(offsets[E+1], sorted_pairs[N])`` where ``sorted_pairs`` holds
    flat pair indices ``t*k + j`` ordered by (expert asc, pair asc) and
    ``offsets`` is the exclusive prefix sum of the per-expert histogram.
    """
    flat = np.asarray(ids).reshape(-1).astype(np.int64)
    sorted_pairs = np.argsort(flat, kind="stable").astype(np.int32)
    counts = np.bincount(flat, minlength=num_experts)
    offsets = np.zeros(num_experts + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts)
    return offsets, sorted_pairs


def grouped_expert_linear(x, wq, scales, biases, group_size: int, expert_ids, act: str):
    """moe.py:8-34: out[n] = rnd(x[n] . dequant(W[ids[n]])^T), in row order."""
    x2 = np.asarray(x, np.float64).reshape(-1, np.shape(x)[-1])
    flat = np.asarray(expert_ids).reshape(-1)
    out = np.zeros((x2.shape[0], wq.shape[-2]), dtype=np.float64)
    for e in np.unique(flat):
        rows = np.nonzero(flat == e)[0]
        w = dequantize(wq[e], scales[e], biases[e], group_size)
        out[rows] = round_act(x2[rows] @ w.T, act)
    return out.reshape(*np.shape(expert_ids), wq.shape[-2])


def silu(v):
    """x * sigmoid(x) in float64, unrounded (the mathematical function)."""
    v = np.asarray(v, np.float64)
    return v / (1.0 + np.exp(-v))


def silu_act(g, act: str) -> np.ndarray:
    """``silu`` of activation.py:21-24 on an act tensor, op by op.

    The reference evaluates the stable form as separate activation-dtype
    ops, each materialising a rounded act tensor:

      e  = exp(-|g|)            (rounded)
      d  = 1 + e                (rounded)
      s  = 1 / d                (rounded)
      sg = where(g < 0, 1 - s, s)   (1 - s rounded)
      silu = g * sg             (rounded)

    Every intermediate here is computed in float64 and rounded once to act.
    For d, 1 - s and g * sg the float64 value is exact (act operands), and
    1 / d is never a rounding tie (d has at most 11 significant bits and is
    not a power of two unless the quotient is exact), so this equals MLX's
    float32-then-act evaluation of each op; exp itself is correctly rounded
    here, MLX's own exp is not pinned.  Consequences of the rounding points:
    for |g| past 8 ln 2 (bf16) or 11 ln 2 (fp16) the rounded 1 + e is 1 and a
    negative g gives exactly 0; for negative g near -3 the rounded 1 - s
    carries a relative error of a few percent against the exact sigmoid.
    """
    g = np.asarray(g, np.float64)
    e = round_act(np.exp(-np.abs(g)), act)
    d = round_act(1.0 + e, act)
    s = round_act(1.0 / d, act)
    sg = np.where(g < 0, round_act(1.0 - s, act), s)
    return round_act(g * sg, act)


def moe_forward(x, weights: dict, top_k: int, norm_topk_prob: bool, act: str, group_size: int):
    """Moe.__call__ (moe.py:69-86).

    ``weights`` holds ``router``, ``gate``, ``up``, ``down`` tuples of
    ``(wq, scales, biases)``.  Returns ``(y, ids, scores)`` with ``y`` of the
    shape of ``x``.
    """
    shape = np.shape(x)
    x2 = np.asarray(x, np.float64).reshape(-1, shape[-1])
    T = x2.shape[0]
    _, _, ids, scores = route_topk(x2, *weights["router"], group_size, top_k, norm_topk_prob, act)
    flat = ids.reshape(-1)
    tok = np.repeat(np.arange(T), top_k)
    H = weights["down"][0].shape[-2]
    down = np.zeros((T * top_k, H), dtype=np.float64)
    for e in np.unique(flat):
        pairs = np.nonzero(flat == e)[0]
        xe = x2[tok[pairs]]
        wg = dequantize(weights["gate"][0][e], weights["gate"][1][e], weights["gate"][2][e], group_size)
        wu = dequantize(weights["up"][0][e], weights["up"][1][e], weights["up"][2][e], group_size)
        wd = dequantize(weights["down"][0][e], weights["down"][1][e], weights["down"][2][e], group_size)
        g = round_act(xe @ wg.T, act)
        u = round_act(xe @ wu.T, act)
        h = round_act(silu_act(g, act) * u, act)
        down[pairs] = round_act(h @ wd.T, act)
    contrib = round_act(down.reshape(T, top_k, H) * scores[..., None], act)
    y = round_act(contrib.sum(axis=1), act)
    return y.reshape(shape), ids.reshape(*shape[:-1], top_k), scores.reshape(*shape[:-1], top_k)


# --------------------------------------------------------------------------
# Seeded synthetic inputs (shared by tests, fixtures and the CPU baseline)
# --------------------------------------------------------------------------


def make_inputs(seed: int, T: int, H: int, E: int, I: int, act: str, group_size: int = 64,
                w_std: float = 0.02, x_std: float = 1.0, router_std: float = 0.02):
    """Seeded activations and MLX-affine-quantised weights.

    x ~ N(0, x_std), router ~ N(0, router_std), experts ~ N(0, w_std), each
    rounded to act before quantisation (the reference quantises fp16/bf16
    weights).  Returns ``(x, weights)`` with ``x`` float64 act values [T, H].
    """
    rng = np.random.default_rng(seed)
    x = round_act(rng.standard_normal((T, H)) * x_std, act)
    wr = round_act(rng.standard_normal((E, H)) * router_std, act)
    wg = round_act(rng.standard_normal((E, I, H)) * w_std, act)
    wu = round_act(rng.standard_normal((E, I, H)) * w_std, act)
    wd = round_act(rng.standard_normal((E, H, I)) * w_std, act)
    weights = {
        "router": quantize(wr, group_size, 4, act),
        "gate": quantize(wg, group_size, 4, act),
        "up": quantize(wu, group_size, 4, act),
        "down": quantize(wd, group_size, 4, act),
    }
    return x, weights


def random_packed(rng, shape, group_size: int, act: str, w_std: float = 0.02):
    """Packed int4 weights of ``shape = (..., out, in)`` drawn directly in the
    quantised domain with the statistics of quantised N(0, w_std) groups:
    codes 7.5 + N(0, 1) * 15 / 4.8 rounded and clipped to [0, 15] (a 64-wide
    normal group spans about 4.8 sigma), signed scales of that range over 15
    steps and biases centring the codes, all act-representable.  Much cheaper
    than quantising a float tensor at the 30B/235B expert shapes, and the same
    layout.

    Each code comes from one uniform byte through an inverse-CDF table; two
    bytes (one uniform 16-bit draw) give the byte holding codes 2i (low
    nibble) and 2i + 1, and four such bytes, little-endian, are one packed
    word, so code 8w + j lands in bits [4j, 4j+4) of word w."""
    *lead, n_out, n_in = shape
    assert n_in % 8 == 0
    nd = statistics.NormalDist()
    table = np.array([min(15.0, max(0.0, round(7.5 + nd.inv_cdf((i + 0.5) / 256) * 15.0 / 4.8)))
                      for i in range(256)], dtype=np.uint8)
    pair = (table[np.arange(65536) & 0xFF] | (table[np.arange(65536) >> 8] << 4)).astype(np.uint8)
    wq = np.empty((*lead, n_out, n_in // 8), dtype=np.uint32)
    flat = wq.reshape(-1, n_in // 8)
    step = max(1, (1 << 24) // n_in)  # rows per batch (bounded temporaries)
    for r in range(0, flat.shape[0], step):
        rows = flat[r:r + step]
        draws = rng.integers(0, 65536, size=(rows.shape[0], n_in // 2), dtype=np.uint16)
        rows[...] = pair[draws].view("<u4")
    gshape = (*lead, n_out, n_in // group_size)
    mag = w_std * 4.8 / 15.0 * (1.0 + 0.1 * rng.standard_normal(gshape))
    sign = np.where(rng.random(gshape) < 0.5, -1.0, 1.0)
    scales = round_act(mag * sign, act)
    biases = round_act(-7.5 * scales + w_std * 0.05 * rng.standard_normal(gshape), act)
    return wq, scales, biases


def make_packed_inputs(seed: int, T: int, H: int, E: int, I: int, act: str,
                       group_size: int = 64, w_std: float = 0.02, x_std: float = 1.0,
                       router_std: float = 0.02):
    """Like :func:`make_inputs`, with the expert weights drawn by
    :func:`random_packed` (the router is still quantised from N(0, router_std)
    so routing follows the reference's quantizer)."""
    rng = np.random.default_rng(seed)
    x = round_act(rng.standard_normal((T, H)) * x_std, act)
    wr = round_act(rng.standard_normal((E, H)) * router_std, act)
    weights = {
        "router": quantize(wr, group_size, 4, act),
        "gate": random_packed(rng, (E, I, H), group_size, act, w_std),
        "up": random_packed(rng, (E, I, H), group_size, act, w_std),
        "down": random_packed(rng, (E, H, I), group_size, act, w_std),
    }
    return x, weights
