"""Committed golden fixtures (tests/golden/*.npz) against the oracle and the HIP path.

CPU: the generator still produces the recorded inputs (SHA-256), and both the
numpy oracle and its C restatement reproduce the recorded outputs.
GPU: routing (logits' ranking, probs, ids, scores) and the dispatch
permutation match bit for bit; the block output is within max-rel 2e-2 and
MAE 1e-3 of the recorded output.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))

import make_golden as G  # noqa: E402
from oracle import moe_oracle as O  # noqa: E402

FIXTURES = sorted(G.CASES)


def _load(name: str) -> dict:
    with np.load(G.HERE / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("name", FIXTURES)
def test_fixture_inputs_are_reproducible(name):
    case = G.CASES[name]
    x, w = G.inputs(case)
    assert str(_load(name)["input_sha256"]) == G.digest(x, w)


@pytest.mark.parametrize("name", FIXTURES)
def test_oracle_reproduces_fixture(name):
    got = G.expected(G.CASES[name])
    ref = _load(name)
    for key in ref:
        assert np.array_equal(got[key], ref[key]), key


@pytest.mark.parametrize("name", FIXTURES)
def test_c_restatement_reproduces_fixture(name):
    from oracle import moe_ref

    case = G.CASES[name]
    act = case["act"]
    x, w = G.inputs(case)
    ref = _load(name)
    layer = moe_ref.Layer(w, act)
    y, ids, scores = moe_ref.forward(O.to_bits(x, act), layer, case["k"], case["norm"], case["gs"])
    assert np.array_equal(np.sort(ids, axis=1), np.sort(ref["ids"], axis=1))
    y_ref = O.from_bits(ref["y"], act)
    d = np.abs(O.from_bits(y, act) - y_ref)
    # both accumulate in float32 (different orders): within a few act ulps
    assert d.max() <= 2e-2 * np.abs(y_ref).max() and d.mean() <= 1e-3


@pytest.mark.gpu
@pytest.mark.parametrize("name", FIXTURES)
def test_hip_path_matches_fixture(name):
    import torch

    from helpers import assert_moe_close, make_moe, qweights, to_act, to_np
    from nano_vllm_metal_amd import moe_dispatch, route_topk

    dev = "cuda:0"
    case = G.CASES[name]
    act, gs, k, norm, T, H = case["act"], case["gs"], case["k"], case["norm"], case["T"], case["H"]
    x, w = G.inputs(case)
    ref = _load(name)
    xt = to_act(x, act, dev)
    probs, ids, scores = route_topk(xt, qweights(w["router"], act, gs, dev), k, norm)
    offsets, pairs = moe_dispatch(ids, case["E"])
    moe = make_moe(w, act, gs, k, norm, dev)
    y = moe(xt.reshape(1, T, H))
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy(), ref["ids"])
    assert np.array_equal(O.to_bits(to_np(probs), act), ref["probs"])
    assert np.array_equal(O.to_bits(to_np(scores), act), ref["scores"])
    assert np.array_equal(offsets.cpu().numpy(), ref["expert_offsets"])
    assert np.array_equal(pairs.cpu().numpy(), ref["sorted_pairs"])
    assert_moe_close(y.reshape(T, H), O.from_bits(ref["y"], act), act, name)
