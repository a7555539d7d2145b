"""Write the committed golden fixtures of the MoE path.

The reference repository stores no vectors for this path (its tests draw
random data at run time and compare with MLX / mlx-lm, which are not
installed here), so these fixtures freeze the oracle's outputs on seeded
inputs:

* ``tiny_moe_f16.npz`` — the tiny parity block: hidden 256, 16 experts, top-4
  renormalised, intermediate 128, 32 tokens, fp16, int4 group 64, seed 1;
* ``ref_moe_f16_g128.npz`` — the shape of tests/test_moe.py:93-131 (hidden 128,
  intermediate 128, 3 experts, top-2, norm_topk_prob, g128), seed 3;
* ``ref_router_f16_g128.npz`` — the shape of tests/test_moe.py:52-90 (4 experts,
  top-2, hidden 128, g128), seed 2.

Inputs are regenerated from ``oracle.moe_oracle.make_inputs(seed, ...)``; each
fixture stores a SHA-256 of the generated inputs so that a change of the
generator is detected instead of silently moving the expected outputs.
Run from the repository root: ``python tests/golden/make_golden.py``.
"""

from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle import moe_oracle as O  # noqa: E402

CASES = {
    "tiny_moe_f16": dict(seed=1, T=32, H=256, E=16, I=128, k=4, norm=True, act="float16", gs=64),
    "ref_moe_f16_g128": dict(seed=3, T=6, H=128, E=3, I=128, k=2, norm=True, act="float16", gs=128),
    "ref_router_f16_g128": dict(seed=2, T=6, H=128, E=4, I=128, k=2, norm=False, act="float16",
                                gs=128),
}


def inputs(case: dict):
    return O.make_inputs(case["seed"], case["T"], case["H"], case["E"], case["I"], case["act"],
                         case["gs"])


def digest(x, weights) -> str:
    h = hashlib.sha256()
    h.update(np.ascontiguousarray(x, np.float64).tobytes())
    for name in ("router", "gate", "up", "down"):
        for a in weights[name]:
            h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def expected(case: dict) -> dict:
    x, w = inputs(case)
    act, gs, k, norm = case["act"], case["gs"], case["k"], case["norm"]
    logits, probs, ids, scores = O.route_topk(x, *w["router"], gs, k, norm, act)
    y, ids_f, scores_f = O.moe_forward(x, w, k, norm, act, gs)
    offsets, pairs = O.dispatch(ids, case["E"])
    return {
        "input_sha256": np.array(digest(x, w)),
        "logits": O.to_bits(logits, act),
        "probs": O.to_bits(probs, act),
        "ids": ids.astype(np.int32),
        "scores": O.to_bits(scores, act),
        "expert_offsets": np.asarray(offsets, np.int32),
        "sorted_pairs": np.asarray(pairs, np.int32),
        "y": O.to_bits(y.reshape(case["T"], case["H"]), act),
    }


def main() -> None:
    for name, case in CASES.items():
        out = expected(case)
        np.savez_compressed(HERE / f"{name}.npz", **out)
        print(name, {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
