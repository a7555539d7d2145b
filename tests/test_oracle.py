"""Pins the CPU oracle (oracle/moe_oracle.py) against facts it does not restate.

Each check is chosen so that a plausible mistake in the oracle (a wrong
nibble order, a transposed operand, a dropped bias, a reversed tie rule, an
off-by-one in the dispatch offsets) fails it:

* rounding: against numpy's own float16 conversion and a float32 bit-level
  bfloat16 rounding, including ties to even;
* packing/dequantisation: hand-packed words and the identity known-answer of
  the reference suite (tests/test_quantized_matmul.py:13-14);
* quantizer: round-trip bound, exact edges, codes in range;
* quantized matmul: exact rational arithmetic (fractions) on a tiny case;
* router: brute force over all orderings of tiny inputs, all-equal logits,
  one-hot logits, renormalised scores summing to one;
* dispatch: brute-force loops, bijection/monotonicity/bincount invariants and
  hypothesis property tests;
* SwiGLU activation: the reference's stable silu form (activation.py:21-24)
  evaluated by torch on the CPU in the activation dtype (a different engine
  whose per-op results are rounded tensors, as MLX's are), plus closed forms
  (the collapse to exactly 0 for large negative inputs, silu(g) = g for large
  positive ones) and its measured distance from the exact function;
* MoE block: a per-token dense loop written independently of moe_forward,
  k = 1 with renormalisation, identical experts;
* the C restatement (oracle/moe_ref.c) against the numpy oracle.
"""

from __future__ import annotations

import itertools
import math
from fractions import Fraction

import numpy as np
import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

from oracle import moe_oracle as O

ACTS = ["float16", "bfloat16"]


def _silu_torch_act(g, act):
    """activation.py:21-24 evaluated by torch on the CPU with act tensors:
    every op of the expression returns a tensor rounded to the act dtype."""
    import torch

    dt = {"float16": torch.float16, "bfloat16": torch.bfloat16}[act]
    x = torch.from_numpy(np.ascontiguousarray(g, dtype=np.float32)).to(dt)
    sig = 1 / (1 + torch.exp(-torch.abs(x)))
    sig = torch.where(x < 0, 1 - sig, sig)
    return (x * sig).double().numpy()


def _all_act_values(act, lo, hi):
    """Every act-representable value in [lo, hi]."""
    b = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    with np.errstate(invalid="ignore"):
        v = O.from_bits(b, act)
    v = v[np.isfinite(v)]
    return np.unique(v[(v >= lo) & (v <= hi)])


# ---------------------------------------------------------------- rounding


def _bf16_round_f32_bits(x32: np.ndarray) -> np.ndarray:
    """RNE to bfloat16 of float32 values by integer arithmetic on the bits."""
    b = x32.astype(np.float32).view(np.uint32).astype(np.uint64)
    lsb = (b >> 16) & 1
    r = ((b + 0x7FFF + lsb) >> 16) << 16
    return r.astype(np.uint32).view(np.float32).astype(np.float64)


def test_round_bf16_matches_bit_rounding_of_float32_values():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(20000) * np.exp(rng.uniform(-20, 20, 20000))).astype(np.float32)
    assert np.array_equal(O.round_act(x.astype(np.float64), "bfloat16"), _bf16_round_f32_bits(x))


def test_round_bf16_ties_to_even():
    # 1 + 2^-8 is halfway between 1 and 1 + 2^-7: ties to the even 1.0;
    # 1 + 3*2^-8 is halfway between 1 + 2^-7 and 1 + 2^-6: ties to 1 + 2^-6
    v = np.array([1 + 2.0 ** -8, 1 + 3 * 2.0 ** -8, -(1 + 2.0 ** -8)])
    assert O.round_act(v, "bfloat16").tolist() == [1.0, 1 + 2.0 ** -6, -1.0]


def test_round_f16_matches_numpy():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(20000) * np.exp(rng.uniform(-12, 10, 20000))
    assert np.array_equal(O.round_act(x, "float16"), x.astype(np.float16).astype(np.float64))


def test_round_is_correct_from_float64_not_via_float32():
    # a float64 value just above a bf16 midpoint whose float32 rounding lands
    # exactly on the midpoint: direct rounding must go up
    mid = 1 + 2.0 ** -8
    v = mid + 2.0 ** -40
    assert O.round_act(np.array([v]), "bfloat16")[0] == 1 + 2.0 ** -7


@pytest.mark.parametrize("act", ACTS)
def test_bits_round_trip(act):
    rng = np.random.default_rng(2)
    v = O.round_act(rng.standard_normal(1000), act)
    assert np.array_equal(O.from_bits(O.to_bits(v, act), act), v)


# ---------------------------------------------------------------- layout


def test_pack_known_word():
    # codes 1..8 in element order -> nibble j holds element j
    assert O.pack_nibbles(np.arange(1, 9)).tolist() == [0x87654321]
    assert O.unpack_nibbles(np.array([0x87654321], np.uint32)).tolist() == list(range(1, 9))


def test_dequantize_closed_form():
    q = np.arange(64) % 16
    wq = O.pack_nibbles(q)[None, :]
    s, b = np.array([[0.5]]), np.array([[-3.0]])
    assert np.array_equal(O.dequantize(wq, s, b, 64)[0], q * 0.5 - 3.0)


@pytest.mark.parametrize("act,gs", [("float16", 128), ("bfloat16", 128), ("bfloat16", 64)])
def test_identity_known_answer(act, gs):
    """eye(N) . dequant(W)^T = dequant(W)^T (test_quantized_matmul.py:13-14)."""
    rng = np.random.default_rng(3)
    w = O.round_act(rng.standard_normal((5, gs)), act)
    wq, s, b = O.quantize(w, gs, 4, act)
    out = O.quantized_matmul(np.eye(gs), wq, s, b, gs, act)
    assert np.array_equal(out, O.round_act(O.dequantize(wq, s, b, gs).T, act))


@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("gs", [64, 128])
def test_quantize_round_trip(act, gs):
    rng = np.random.default_rng(4)
    w = O.round_act(rng.standard_normal((7, 3 * gs)) * 0.02, act)
    wq, s, b = O.quantize(w, gs, 4, act)
    assert wq.dtype == np.uint32 and wq.shape == (7, 3 * gs // 8)
    codes = O.unpack_nibbles(wq)
    assert codes.max() <= 15
    deq = O.dequantize(wq, s, b, gs)
    err = np.abs(deq - w).reshape(7, 3, gs)
    # The zero-point adjustment (scale = edge / round(edge / scale)) moves the
    # scale by at most 0.5/7.5 of itself (|edge| >= 7.5 steps), so the far edge
    # may miss by up to one step: error <= 1.5 steps, plus act rounding of
    # scale and bias.
    sa, ba = np.abs(s)[..., None], np.abs(b)[..., None]
    bound = 1.5 * sa * (1 + 2 ** -7) + 15 * sa * 2 ** -7 + ba * 2 ** -7 + 1e-12
    assert np.all(err <= bound)
    # the edge with the larger magnitude is exact (code 0 -> bias)
    assert np.all(np.abs(deq.reshape(7, 3, gs) - w.reshape(7, 3, gs)).min(axis=-1) <= ba[..., 0] * 2 ** -7)


def test_quantize_constant_group_is_exact():
    w = np.full((1, 64), 0.25)
    wq, s, b = O.quantize(w, 64, 4, "bfloat16")
    assert np.array_equal(O.dequantize(wq, s, b, 64), w)


def test_quantized_matmul_exact_rational():
    """Tiny case against exact fractions: catches a transposed operand or a
    dropped bias."""
    act, gs = "bfloat16", 64
    rng = np.random.default_rng(5)
    a = O.round_act(rng.standard_normal((2, 128)), act)
    w = O.round_act(rng.standard_normal((3, 128)), act)
    wq, s, b = O.quantize(w, gs, 4, act)
    q = O.unpack_nibbles(wq)
    out = O.quantized_matmul(a, wq, s, b, gs, act)
    for i in range(2):
        for k in range(3):
            tot = Fraction(0)
            for d in range(128):
                wd = Fraction(int(q[k, d])) * Fraction(s[k, d // gs]) + Fraction(b[k, d // gs])
                tot += Fraction(a[i, d]) * wd
            assert out[i, k] == O.round_act(np.array([float(tot)]), act)[0]


# ---------------------------------------------------------------- router


def _brute_topk(probs_row, k):
    order = sorted(range(len(probs_row)), key=lambda e: (-probs_row[e], e))
    return order[:k]


@pytest.mark.parametrize("act", ACTS)
def test_topk_brute_force_with_ties(act):
    rng = np.random.default_rng(6)
    for _ in range(200):
        E, k = 6, 3
        # few distinct values so ties are frequent
        probs = O.round_act(rng.integers(0, 4, E) / 8.0, act)
        ids = O.topk_lower_index(probs[None], k)[0].tolist()
        assert ids == _brute_topk(probs.tolist(), k)
        # exhaustive check: no other k-subset has a strictly better sorted key
        best = min(itertools.combinations(range(E), k),
                   key=lambda c: sorted((-probs[e], e) for e in c))
        assert sorted(ids) == sorted(best)


def test_route_all_equal_logits_pick_lowest_experts():
    x = np.ones((3, 64))
    wr = np.zeros((16, 64))
    wq, s, b = O.quantize(wr, 64, 4, "bfloat16")
    _, probs, ids, scores = O.route_topk(x, wq, s, b, 64, 4, True, "bfloat16")
    assert ids.tolist() == [[0, 1, 2, 3]] * 3
    assert np.all(probs == O.round_act(np.array([1 / 16]), "bfloat16")[0])
    assert np.all(scores == 0.25)


def test_route_one_hot_logit():
    x = np.ones((1, 64))
    wr = np.zeros((8, 64))
    wr[5] = 0.125  # logit 8 for expert 5
    wq, s, b = O.quantize(wr, 64, 4, "bfloat16")
    logits, probs, ids, scores = O.route_topk(x, wq, s, b, 64, 2, False, "bfloat16")
    assert logits[0, 5] == 8.0 and np.all(np.delete(logits[0], 5) == 0)
    assert ids[0].tolist() == [5, 0]
    p5 = math.exp(8) / (math.exp(8) + 7)
    assert scores[0, 0] == O.round_act(np.array([p5]), "bfloat16")[0]


@pytest.mark.parametrize("act", ACTS)
def test_renormalised_scores_sum_to_one(act):
    x, w = O.make_inputs(7, 64, 256, 16, 64, act)
    _, _, ids, sc = O.route_topk(x, *w["router"], 64, 4, True, act)
    ulp = 2.0 ** (-7 if act == "bfloat16" else -10)
    assert np.all(np.abs(sc.sum(axis=1) - 1) <= 4 * ulp)
    assert np.all(np.diff(sc, axis=1) <= 0)  # slots in probability order


def test_softmax_invariants():
    rng = np.random.default_rng(8)
    lg = O.round_act(rng.standard_normal((50, 32)) * 3, "bfloat16")
    p = O.softmax_act(lg, "bfloat16")
    assert np.all(np.abs(p.sum(axis=1) - 1) < 32 * 2 ** -8)
    # monotone: larger logit never gets a smaller probability
    for r in range(50):
        o = np.argsort(lg[r])
        assert np.all(np.diff(p[r][o]) >= 0)


# ---------------------------------------------------------------- dispatch


def _brute_dispatch(ids, E):
    sorted_pairs, offsets = [], [0]
    for e in range(E):
        sorted_pairs += [p for p, v in enumerate(ids) if v == e]
        offsets.append(len(sorted_pairs))
    return offsets, sorted_pairs


def test_dispatch_brute_force():
    rng = np.random.default_rng(9)
    for n, E in [(0, 4), (1, 1), (37, 5), (200, 16)]:
        ids = rng.integers(0, E, n)
        off, srt = O.dispatch(ids, E)
        bo, bs = _brute_dispatch(ids.tolist(), E)
        assert off.tolist() == bo and srt.tolist() == bs


@settings(max_examples=100, deadline=None)
@given(st.lists(st.integers(0, 9), max_size=300), st.integers(10, 12))
def test_dispatch_properties(ids, E):
    ids = np.array(ids, dtype=np.int64)
    off, srt = O.dispatch(ids, E)
    assert sorted(srt.tolist()) == list(range(len(ids)))  # bijection
    assert np.all(np.diff(ids[srt]) >= 0) if len(ids) else True  # expert-major
    assert np.array_equal(np.diff(off), np.bincount(ids, minlength=E))
    for e in range(E):  # stable inside each expert
        assert np.all(np.diff(srt[off[e]:off[e + 1]]) > 0)


# ---------------------------------------------------------------- packed generator


def test_random_packed_layout_and_codes():
    """Codes of the packed-domain generator: code 8w + j of a row sits in bits
    [4j, 4j + 4) of word w, each drawn from one uniform byte through the
    inverse-CDF table (byte i -> round(7.5 + Phi^-1((i + .5) / 256) * 15 / 4.8))."""
    import statistics

    nd = statistics.NormalDist()
    table = np.array([min(15, max(0, round(7.5 + nd.inv_cdf((i + 0.5) / 256) * 15 / 4.8)))
                      for i in range(256)])
    wq, s, b = O.random_packed(np.random.default_rng(5), (3, 7, 128), 64, "bfloat16")
    draws = np.random.default_rng(5).integers(0, 65536, size=(21, 64), dtype=np.uint16)
    codes = np.stack([table[draws & 0xFF], table[draws >> 8]], axis=-1).reshape(3, 7, 128)
    assert np.array_equal(O.unpack_nibbles(wq), codes)
    assert s.shape == b.shape == (3, 7, 2)
    assert np.array_equal(O.round_act(s, "bfloat16"), s) and np.all(s != 0)


# ---------------------------------------------------------------- SwiGLU activation


@pytest.mark.parametrize("act", ACTS)
def test_silu_act_matches_per_op_act_evaluation(act):
    """Every act value in [-16, 16]: the oracle's op-by-op silu equals the
    reference expression evaluated with torch act tensors, except where the
    two exp implementations round a value lying within float32 error of an
    act rounding tie."""
    g = _all_act_values(act, -16.0, 16.0)
    got = O.silu_act(g, act)
    ref = _silu_torch_act(g, act)
    diff = got != ref
    assert diff.mean() < 2e-3, (act, int(diff.sum()), g[diff][:10])
    # a mismatch is one act ulp at most
    ulp = np.abs(ref) * 2.0 ** -(7 if act == "bfloat16" else 10)
    assert np.all(np.abs(got - ref)[diff] <= ulp[diff] + 1e-30)


@pytest.mark.parametrize("act,edge", [("bfloat16", 8), ("float16", 11)])
def test_silu_act_closed_forms(act, edge):
    """1 + exp(-|g|) rounds to 1 once exp(-|g|) is below half an act ulp of 1
    (|g| > edge * ln 2): the reference's sigmoid is then exactly 1 or 0, so
    silu(g) = g for positive g and exactly 0 for negative g."""
    g = _all_act_values(act, -60.0, 60.0)
    far = np.abs(g) > edge * math.log(2.0) + 0.05
    y = O.silu_act(g, act)
    assert np.all(y[far & (g > 0)] == g[far & (g > 0)])
    assert np.all(y[far & (g < 0)] == 0.0)
    assert O.silu_act(np.array([0.0]), act)[0] == 0.0
    # the exact function is not zero there: the rounding points matter
    assert np.all(O.silu(g[far & (g < 0) & (g > -20)]) < 0)


@pytest.mark.parametrize("act", ACTS)
def test_silu_act_distance_from_exact(act):
    """Positive inputs stay within two act ulps of the exact silu; negative
    ones carry the error of the rounded 1 - s, largest near g = -3 (several
    percent in bfloat16), which a single-rounding silu would not show."""
    g = _all_act_values(act, -8.0, 8.0)
    y = O.silu_act(g, act)
    ex = O.silu(g)
    pos = g > 2.0 ** -13  # (below, silu(g) ~ g/2 is subnormal in float16)
    ulp = 2.0 ** -(7 if act == "bfloat16" else 10)
    assert np.all(np.abs(y - ex)[pos] <= 2 * ulp * np.abs(ex)[pos])
    band = (g > -4) & (g < -2)
    rel = np.abs(y - ex)[band] / np.abs(ex)[band]
    if act == "bfloat16":
        assert rel.max() > 0.01
    single = O.round_act(ex, act)
    assert np.any(single[g < 0] != y[g < 0])


# ---------------------------------------------------------------- MoE block


def _dense_reference(x, w, k, norm, act, gs):
    """Per-token loop over slots, written without the oracle's batching."""
    T = x.shape[0]
    _, _, ids, scores = O.route_topk(x, *w["router"], gs, k, norm, act)
    y = np.zeros_like(x)
    for t in range(T):
        acc = 0.0
        terms = []
        for j in range(k):
            e = ids[t, j]
            g = O.round_act(O.dequantize(w["gate"][0][e], w["gate"][1][e], w["gate"][2][e], gs) @ x[t], act)
            u = O.round_act(O.dequantize(w["up"][0][e], w["up"][1][e], w["up"][2][e], gs) @ x[t], act)
            h = O.round_act(_silu_torch_act(g, act) * u, act)
            d = O.round_act(O.dequantize(w["down"][0][e], w["down"][1][e], w["down"][2][e], gs) @ h, act)
            terms.append(O.round_act(d * scores[t, j], act))
        y[t] = O.round_act(np.sum(terms, axis=0), act)
    return y, ids, scores


@pytest.mark.parametrize("act", ACTS)
def test_moe_forward_matches_dense_loop(act):
    x, w = O.make_inputs(10, 6, 128, 8, 64, act)
    y, ids, sc = O.moe_forward(x, w, 3, True, act, 64)
    yd, idd, scd = _dense_reference(x, w, 3, True, act, 64)
    assert np.array_equal(ids, idd) and np.array_equal(sc, scd)
    assert np.array_equal(y, yd)


def test_moe_top1_renorm_is_expert_output():
    act = "bfloat16"
    x, w = O.make_inputs(11, 5, 128, 4, 64, act)
    y, ids, sc = O.moe_forward(x, w, 1, True, act, 64)
    assert np.all(sc == 1.0)
    for t in range(5):
        e = ids[t, 0]
        g = O.grouped_expert_linear(x[t:t + 1], *w["gate"], 64, np.array([e]), act)
        u = O.grouped_expert_linear(x[t:t + 1], *w["up"], 64, np.array([e]), act)
        h = O.round_act(_silu_torch_act(g, act) * u, act)
        d = O.grouped_expert_linear(h, *w["down"], 64, np.array([e]), act)
        assert np.array_equal(y[t], d[0])


def test_moe_identical_experts():
    act = "float16"
    x, w = O.make_inputs(12, 4, 128, 4, 64, act)
    for name in ("gate", "up", "down"):
        wq, s, b = w[name]
        w[name] = (np.repeat(wq[:1], 4, 0), np.repeat(s[:1], 4, 0), np.repeat(b[:1], 4, 0))
    y, _, sc = O.moe_forward(x, w, 2, True, act, 64)
    one, _, _ = O.moe_forward(x, w, 1, True, act, 64)
    # sum_j rnd(d * s_j) with sum s_j ~ 1 reproduces the single-expert output
    assert np.max(np.abs(y - one)) <= 4 * 2.0 ** -10 * np.max(np.abs(one)) + 1e-6


def test_grouped_expert_linear_row_order():
    act = "bfloat16"
    rng = np.random.default_rng(13)
    x = O.round_act(rng.standard_normal((2, 3, 64)), act)
    wq, s, b = O.quantize(O.round_act(rng.standard_normal((3, 16, 64)) * 0.1, act), 64, 4, act)
    ids = np.array([[2, 0, 1], [1, 2, 0]])
    out = O.grouped_expert_linear(x, wq, s, b, 64, ids, act)
    for i in range(2):
        for j in range(3):
            ref = O.round_act(O.dequantize(wq[ids[i, j]], s[ids[i, j]], b[ids[i, j]], 64) @ x[i, j], act)
            assert np.array_equal(out[i, j], ref)


# ---------------------------------------------------------------- C restatement


@pytest.mark.parametrize("act,shape", [("float16", (32, 256, 16, 128, 4)),
                                       ("bfloat16", (16, 512, 32, 128, 8))])
def test_c_restatement_matches_numpy_oracle(act, shape):
    from oracle import moe_ref as R

    T, H, E, I, k = shape
    x, w = O.make_inputs(14, T, H, E, I, act)
    y, ids, sc = O.moe_forward(x, w, k, True, act, 64)
    yc, idc, scc = R.forward(R.bits(x, act), R.Layer(w, act), k, True, 64)
    assert np.array_equal(idc, ids)
    assert np.array_equal(O.from_bits(scc, act), sc)
    d = np.abs(O.from_bits(yc, act) - y)
    # the C path accumulates expert products in float32 (the reference's own
    # CPU loop), the numpy oracle in float64
    assert d.max() <= 2e-2 * np.abs(y).max() and d.mean() <= 1e-4


def test_c_dispatch_matches_numpy():
    from oracle import moe_ref as R

    rng = np.random.default_rng(15)
    ids = rng.integers(0, 64, 5000).astype(np.int32)
    off, srt = R.dispatch(ids, 64)
    o2, s2 = O.dispatch(ids, 64)
    assert np.array_equal(off, o2) and np.array_equal(srt, s2)
