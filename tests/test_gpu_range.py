"""Activations beyond fp16's range through the prefill path of nvm_moe_forward.

The prefill GEMMs multiply fp16 copies of x and h.  bf16 reaches 2^127, fp16
only 65504, so the copies carry a power-of-two shift per row and 64-value
group (bf16_to_f16_pairs) that the GEMMs undo on their float32 sums.  These
cases send through the forward, at the 30B-A3B shape in the prefill regime:

* rows of x scaled by 2^17 (|x| up to ~5e5), and normal rows with a few
  columns at +-3e5 (one shifted group among unshifted ones);
* rows of x scaled by 300 (x itself inside fp16's range), whose gate/up sums
  make |h| well above 65504, so that h's groups are shifted;
* rows whose values span more than 40 binades (2^-40 .. 2^20 around N(0,1));

for the int8 router's batches (T >= 128: it writes the fp16 copy of x) and
for smaller batches (the separate conversion launch).  Router ids and scores
must equal the oracle's bit for bit; the outputs must meet the block
tolerance row by row (relative to each row's largest reference value) and
the reference suite's elementwise allclose.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import ALLCLOSE, MAX_REL, make_moe, to_act, to_np
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _wide_x(seed, T, H, act):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, H))
    x[0:8] *= 2.0 ** 17                                    # whole rows beyond fp16
    cols = rng.choice(H, size=(8, 3), replace=False)
    for r in range(8):                                     # single large columns
        x[8 + r, cols[r]] = 3e5 * np.sign(rng.standard_normal(3))
    x[16:24] *= 300.0                                      # |h| beyond fp16
    x[24:32] *= 2.0 ** rng.integers(-40, 21, size=(8, H))  # > 40 binades a row
    return O.round_act(x, act)


@pytest.mark.parametrize("T", [512, 96])
def test_prefill_operands_beyond_fp16_range(T):
    act, H, E, I, gs, k = "bfloat16", 2048, 128, 768, 64, 8
    _, w = O.make_packed_inputs(500 + T, 1, H, E, I, act, gs)
    x = _wide_x(501 + T, T, H, act)
    moe = make_moe(w, act, gs, k, True, DEV)
    moe.regime = "prefill"
    y, ids, scores = moe.forward(to_act(x, act, DEV), return_routing=True)
    torch.cuda.synchronize()
    rows = np.r_[0:40, T - 8:T]
    y_ref, ids_ref, sc_ref = O.moe_forward(x[rows], w, k, True, act, gs)
    assert np.array_equal(ids.cpu().numpy()[rows], ids_ref), "ids differ"
    assert np.array_equal(to_np(scores)[rows], sc_ref), "scores differ"
    yy = to_np(y)[rows]
    assert np.all(np.isfinite(yy)), "non-finite output"
    # the large rows' outputs are far beyond fp16's range: the shifts took effect
    assert np.abs(yy[:8]).max() > 65504.0 and np.abs(yy[16:24]).max() > 65504.0
    d = np.abs(yy - y_ref)
    scale = np.maximum(np.abs(y_ref).max(axis=1), 1e-30)
    row_rel = d.max(axis=1) / scale
    row_mae = d.mean(axis=1) / scale
    print(f"T={T}: worst row max-rel {row_rel.max():.3e}, worst row mean-rel "
          f"{row_mae.max():.3e}", flush=True)
    assert row_rel.max() <= MAX_REL, row_rel
    assert row_mae.max() <= 1e-3, row_mae
    rtol, atol = ALLCLOSE[act]
    bad = ~np.isclose(yy, y_ref, rtol=rtol, atol=atol * scale[:, None])
    assert not bad.any(), f"{int(bad.sum())} elements outside allclose"
