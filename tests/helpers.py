"""Shared helpers of the test suite: oracle arrays <-> device tensors, tolerances."""

from __future__ import annotations

import numpy as np
import torch

TORCH_ACT = {"float16": torch.float16, "bfloat16": torch.bfloat16}

# Tolerance of the MoE output against fp32-accumulated reference results:
# max error relative to the largest reference magnitude, and mean absolute
# error (for outputs of unit scale, mean error relative to that magnitude).
MAX_REL = 2e-2
MAE = 1e-3
# the reference suite's own assert_allclose tolerances (tests/utils.py:25-35)
ALLCLOSE = {"float16": (5e-2, 1e-3), "bfloat16": (5e-2, 1e-2)}


def to_act(a, act: str, device) -> torch.Tensor:
    """float64 act-representable values -> act tensor (exact)."""
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(TORCH_ACT[act]).to(device)


def to_words(wq, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(wq, dtype=np.uint32).view(np.int32)).to(device)


def qweights(t3, act: str, group_size: int, device):
    from nano_vllm_metal_amd import QuantizedWeights

    wq, s, b = t3
    return QuantizedWeights(to_act(s, act, device), to_act(b, act, device), group_size, 4,
                            to_words(wq, device))


def make_moe(weights: dict, act: str, group_size: int, top_k: int, norm: bool, device):
    from nano_vllm_metal_amd import Moe

    return Moe(qweights(weights["router"], act, group_size, device),
               qweights(weights["gate"], act, group_size, device),
               qweights(weights["up"], act, group_size, device),
               qweights(weights["down"], act, group_size, device),
               num_experts_per_tok=top_k, norm_topk_prob=norm)


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def assert_moe_close(y, y_ref, act: str, what: str = "", mae_rel: bool = False) -> dict:
    y = to_np(y) if isinstance(y, torch.Tensor) else np.asarray(y, np.float64)
    y_ref = np.asarray(y_ref, np.float64)
    assert y.shape == y_ref.shape, (y.shape, y_ref.shape)
    d = np.abs(y - y_ref)
    scale = max(float(np.abs(y_ref).max()), 1e-30)
    stats = {"max_rel": float(d.max()) / scale,
             "mae": float(d.mean()) / (scale if mae_rel else 1.0), "max_abs": float(d.max())}
    assert np.all(np.isfinite(y)), f"{what}: non-finite output"
    assert stats["max_rel"] <= MAX_REL, f"{what}: max rel err {stats}"
    assert stats["mae"] <= MAE, f"{what}: mean abs err {stats}"
    rtol, atol = ALLCLOSE[act]
    bad = ~np.isclose(y, y_ref, rtol=rtol, atol=atol)
    assert not bad.any(), f"{what}: {int(bad.sum())} elements outside allclose, {stats}"
    return stats
