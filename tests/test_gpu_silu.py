"""SwiGLU of the expert products at every activation value.

silu (activation.py:21-24) is evaluated op by op in the activation dtype,
each intermediate rounded: e = exp(-|g|), d = 1 + e, s = 1 / d,
sg = 1 - s for g < 0, silu = g * sg.  The kernels take exp and 1/d from the
hardware's fast float32 instructions before rounding them, so they equal the
correctly rounded ops only if no input lands close enough to a rounding
boundary for those instructions' error to matter.  The input of silu is an
activation value (the gate product rounded), so there are at most 65536 of
them: this sends every one through the gate/up products and compares h bit
for bit with the oracle's op-by-op silu (each op computed in float64 and
rounded once).

The gate product is made equal to a chosen value v exactly: x is one-hot on
hidden column 0, every code and scale is zero, and the bias of group 0 of
gate row i is v (so the product is 1 * v); the up product is 1 the same way,
so h = rnd(silu(v) * 1).  Token t goes to expert t alone (top-k 1).  The
decode products (exact codes, no weight rounding) take every finite value;
the prefill GEMM rounds each dequantised weight to fp16, so there the values
are those fp16 holds exactly.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from nano_vllm_metal_amd import _lib
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _all_values(act: str) -> np.ndarray:
    """Every finite value of the activation dtype, as float64."""
    bits = np.arange(1 << 16, dtype=np.uint32)
    with np.errstate(invalid="ignore"):
        if act == "bfloat16":
            v = (bits << 16).view(np.float32).astype(np.float64)
        else:
            v = bits.astype(np.uint16).view(np.float16).astype(np.float64)
    return v[np.isfinite(v)]


@pytest.mark.parametrize("act", ["bfloat16", "float16"])
@pytest.mark.parametrize("regime", ["decode", "prefill"])
def test_swiglu_at_every_gate_value(act, regime):
    vals = _all_values(act)
    if regime == "prefill":
        # values the GEMM's fp16 weights hold exactly
        with np.errstate(over="ignore"):
            vals = vals[vals.astype(np.float16).astype(np.float64) == vals]
    E, I, H, gs = 64, 1024, 768, 64
    n = E * I
    v = np.zeros(n)
    v[: min(n, vals.size)] = vals[:n]
    rest = vals[n:]
    rounds = [v]
    while rest.size:
        w = np.zeros(n)
        w[: min(n, rest.size)] = rest[:n]
        rounds.append(w)
        rest = rest[n:]
    dt = torch.bfloat16 if act == "bfloat16" else torch.float16
    lib = _lib.load()
    T = E
    x = torch.zeros((T, H), dtype=dt, device=DEV)
    x[:, 0] = 1.0
    zeros_w = torch.zeros((E, I, H // 8), dtype=torch.int32, device=DEV)
    zeros_s = torch.zeros((E, I, H // gs), dtype=dt, device=DEV)
    bu = torch.zeros((E, I, H // gs), dtype=dt, device=DEV)
    bu[:, :, 0] = 1.0
    offsets = torch.arange(E + 1, dtype=torch.int32, device=DEV)
    pairs = torch.arange(T, dtype=torch.int32, device=DEV)
    h = torch.empty((T, I), dtype=dt, device=DEV)
    reg = _lib.REGIME_DECODE if regime == "decode" else _lib.REGIME_PREFILL
    bad_total = 0
    for vr in rounds:
        bg = torch.zeros((E, I, H // gs), dtype=dt, device=DEV)
        bg[:, :, 0] = torch.from_numpy(vr.reshape(E, I)).to(dt).to(DEV)
        _lib.check(lib.nvm_moe_expert_gateup(
            x.data_ptr(), T, H, I, E, 1, gs, 4, _lib.dtype_code(dt), zeros_w.data_ptr(),
            zeros_s.data_ptr(), bg.data_ptr(), zeros_w.data_ptr(), zeros_s.data_ptr(),
            bu.data_ptr(), offsets.data_ptr(), pairs.data_ptr(), h.data_ptr(), reg,
            _lib.stream_of(torch.device(DEV))))
        torch.cuda.synchronize()
        got = h.float().cpu().numpy().astype(np.float64).reshape(-1)
        want = O.round_act(O.silu_act(vr, act) * 1.0, act)
        same = (got == want) | (np.isnan(got) & np.isnan(want))
        bad = np.flatnonzero(~same)
        if bad.size:
            print(f"{act} {regime}: {bad.size} of {vr.size} differ, e.g. g={vr[bad[:5]]} "
                  f"got {got[bad[:5]]} want {want[bad[:5]]}", flush=True)
        bad_total += bad.size
    assert bad_total == 0
