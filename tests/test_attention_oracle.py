"""Pins of the paged-attention oracle (oracle/attention_oracle.py), on the CPU.

Each check is a closed form or an invariant that a plausible mistake in the
restatement (kv-head mapping, slot/page indexing, causal offset, skipped
pages, int8 scales) would break; none re-types the oracle's own formula.
The scenarios follow the reference's tests/test_paged_attention.py:105-188.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import attention_oracle as AO


def _case(seed, B=2, Hq=4, Hkv=2, L=1, D=8, ps=4, P=6, mp=3):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B * Hq, L, D))
    kp, vp = AO.make_pool(rng, P, Hkv, ps, D)
    bt = np.stack([rng.permutation(P)[:mp] for _ in range(B)]).astype(np.int32)
    return rng, q, kp, vp, bt


def test_single_visible_position_returns_its_value():
    rng, q, kp, vp, bt = _case(1)
    lens = np.array([1, 1], np.int32)
    out = AO.paged_attention(q, kp, vp, bt, lens, 0.3, False, 2, 4)
    for n in range(8):
        b, kvh = n // 4, (n % 4) // 2
        assert np.allclose(out[n, 0], vp[bt[b, 0], kvh, 0])


def test_identical_keys_average_the_values():
    rng, q, kp, vp, bt = _case(2)
    kp[:] = kp[0, 0, 0]
    lens = np.array([7, 12], np.int32)
    out = AO.paged_attention(q, kp, vp, bt, lens, 0.5, False, 2, 4)
    for n in range(8):
        b, kvh = n // 4, (n % 4) // 2
        rows = [vp[bt[b, j // 4], kvh, j % 4] for j in range(lens[b])]
        assert np.allclose(out[n, 0], np.mean(rows, axis=0))


@pytest.mark.parametrize("L,causal", [(1, False), (1, True), (3, True), (3, False)])
def test_matches_dense_attention_over_gathered_pages(L, causal):
    """test_paged_attention.py:105-138: paged == dense over the gathered K/V."""
    rng, q, kp, vp, bt = _case(3, L=L)
    lens = np.array([6, 11], np.int32)
    out = AO.paged_attention(q, kp, vp, bt, lens, 0.35, causal, 2, 4)
    for n in range(8):
        b, kvh = n // 4, (n % 4) // 2
        keys = np.stack([kp[bt[b, j // 4], kvh, j % 4] for j in range(lens[b])])
        vals = np.stack([vp[bt[b, j // 4], kvh, j % 4] for j in range(lens[b])])
        ref = AO.dense_attention(q[n], keys, vals, 0.35, causal)
        assert np.allclose(out[n], ref)


def test_empty_request_and_missing_pages():
    """test_paged_attention.py:140-188: context 0 -> zeros; a page id of -1 (or
    past the pool) skips its positions; capacity caps the context."""
    rng, q, kp, vp, bt = _case(4)
    lens = np.array([0, 9], np.int32)
    bt[1, 1] = -1
    out = AO.paged_attention(q, kp, vp, bt, lens, 0.4, False, 2, 4)
    assert np.all(out[:4] == 0)
    for n in range(4, 8):
        kvh = (n % 4) // 2
        pos = [0, 1, 2, 3, 8]  # page 1 (positions 4..7) skipped
        keys = np.stack([kp[bt[1, j // 4], kvh, j % 4] for j in pos])
        vals = np.stack([vp[bt[1, j // 4], kvh, j % 4] for j in pos])
        assert np.allclose(out[n], AO.dense_attention(q[n], keys, vals, 0.4, False))
    bt2 = bt.copy()
    bt2[1, 1] = kp.shape[0] + 3
    assert np.allclose(AO.paged_attention(q, kp, vp, bt2, lens, 0.4, False, 2, 4), out)
    big = np.array([0, 1000], np.int32)  # capacity 3 pages * 4 slots
    full = AO.paged_attention(q, kp, vp, bt, np.array([0, 12], np.int32), 0.4, False, 2, 4)
    assert np.allclose(AO.paged_attention(q, kp, vp, bt, big, 0.4, False, 2, 4), full)


def test_page_permutation_invariance():
    rng, q, kp, vp, bt = _case(5)
    lens = np.array([10, 5], np.int32)
    out = AO.paged_attention(q, kp, vp, bt, lens, 0.25, False, 2, 4)
    perm = rng.permutation(kp.shape[0])            # physical page i -> perm[i]
    kp2, vp2 = np.empty_like(kp), np.empty_like(vp)
    kp2[perm], vp2[perm] = kp, vp
    assert np.allclose(AO.paged_attention(q, kp2, vp2, perm[bt], lens, 0.25, False, 2, 4), out)


def test_grouped_heads_equal_repeated_kv_heads():
    """num_kv_heads < num_heads equals the same pages with each kv head
    repeated for its query-head group."""
    rng, q, kp, vp, bt = _case(6, Hq=6, Hkv=2)
    lens = np.array([9, 4], np.int32)
    out = AO.paged_attention(q, kp, vp, bt, lens, 0.3, False, 2, 6)
    kp3, vp3 = np.repeat(kp, 3, axis=1), np.repeat(vp, 3, axis=1)
    assert np.allclose(AO.paged_attention(q, kp3, vp3, bt, lens, 0.3, False, 6, 6), out)


def test_causal_rows_equal_single_row_calls():
    """Row i of a causal L-row call sees the context of a one-row call with
    context_len - L + i + 1 positions."""
    rng, q, kp, vp, bt = _case(7, L=4)
    lens = np.array([7, 12], np.int32)
    out = AO.paged_attention(q, kp, vp, bt, lens, 0.45, True, 2, 4)
    for i in range(4):
        one = AO.paged_attention(q[:, i:i + 1], kp, vp, bt, lens - 4 + i + 1, 0.45, False, 2, 4)
        assert np.allclose(out[:, i], one[:, 0])


def test_int8_pages_equal_float_pages_of_code_times_scale():
    rng, q, kp, vp, bt = _case(8)
    kc, ksc = AO.quantize_int8(kp)
    vc, vsc = AO.quantize_int8(vp)
    lens = np.array([8, 11], np.int32)
    out = AO.paged_attention(q, kc, vc, bt, lens, 0.3, False, 2, 4, ksc, vsc)
    kf = kc.astype(np.float64) * ksc[..., None]
    vf = vc.astype(np.float64) * vsc[..., None]
    assert np.allclose(AO.paged_attention(q, kf, vf, bt, lens, 0.3, False, 2, 4), out)
    # the quantiser: |x - code*scale| <= scale/2 and codes within [-127, 127]
    assert np.all(np.abs(kp - kf) <= ksc[..., None] / 2 + 1e-6)
    assert np.abs(kc.astype(int)).max() <= 127
