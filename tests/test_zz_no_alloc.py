"""nvm_moe_forward_noalloc against nvm_moe_forward, through the C ABI.

The allocation-free entry point runs the same kernels on a static device
array instead of a caller workspace, so its outputs must be bit-identical to
the workspace entry point's: two calls in a row (the second smaller, on the
array the first one left behind), decode and prefill regimes, and the
rejection of a batch whose workspace exceeds the array.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from helpers import make_moe, to_act
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _args(moe, x):
    from nano_vllm_metal_amd import _lib

    T, H = x.shape
    E, I = moe.check_operands(x.dtype, H)
    ops = moe._operands()
    flat = [t.data_ptr() for trio in ops for t in trio]
    head = [x.data_ptr(), T, H, I, E, moe.num_experts_per_tok, int(moe.norm_topk_prob),
            moe.w_gate.group_size, moe.w_gate.bits, _lib.dtype_code(x.dtype)]
    return head, flat, ops


def _run_both(moe, x, regime):
    from nano_vllm_metal_amd import _lib

    lib = _lib.load()
    T, H = x.shape
    k = moe.num_experts_per_tok
    head, flat, ops = _args(moe, x)
    st = _lib.stream_of(x.device)
    size = ctypes.c_size_t()
    _lib.check(lib.nvm_moe_workspace_size(T, H, head[3], head[4], k, ctypes.byref(size)))
    ws = torch.empty(size.value, dtype=torch.uint8, device=x.device)
    y0 = torch.empty_like(x)
    ids0 = torch.empty((T, k), dtype=torch.int32, device=x.device)
    sc0 = torch.empty((T, k), dtype=x.dtype, device=x.device)
    _lib.check(lib.nvm_moe_forward(*head, *flat, y0.data_ptr(), ids0.data_ptr(), sc0.data_ptr(),
                                   regime, ws.data_ptr(), ws.numel(), st))
    y1 = torch.full_like(x, float("nan"))
    ids1 = torch.full((T, k), -7, dtype=torch.int32, device=x.device)
    sc1 = torch.full((T, k), float("nan"), dtype=x.dtype, device=x.device)
    _lib.check(lib.nvm_moe_forward_noalloc(*head, *flat, y1.data_ptr(), ids1.data_ptr(),
                                           sc1.data_ptr(), regime, st))
    torch.cuda.synchronize()
    del ops
    return (y0, ids0, sc0), (y1, ids1, sc1), size.value


def _case(seed, T, H=2048, E=128, I=768, act="bfloat16"):
    x, w = O.make_packed_inputs(seed, T, H, E, I, act, 64)
    return to_act(x, act, DEV), make_moe(w, act, 64, 8, True, DEV)


@pytest.mark.parametrize("T1,T2,regime", [(64, 8, 0), (300, 33, 2)])
def test_noalloc_matches_workspace_entry_point(T1, T2, regime):
    """Two calls in a row on the shared array, the second smaller."""
    from nano_vllm_metal_amd import _lib

    lib = _lib.load()
    cap = ctypes.c_size_t()
    _lib.check(lib.nvm_moe_scratch_bytes(ctypes.byref(cap)))
    x, moe = _case(41, T1)
    for T in (T1, T2):
        a, b, need = _run_both(moe, x[:T].contiguous(), regime)
        print(f"noalloc T={T} regime={regime}: workspace {need} of {cap.value} bytes", flush=True)
        assert need <= cap.value
        for u, v, what in zip(a, b, ("y", "ids", "scores")):
            assert torch.equal(u, v), f"T={T}: {what} differs from nvm_moe_forward"


def test_noalloc_rejects_batches_beyond_the_array():
    """A batch whose workspace exceeds the static array is refused with
    NVM_ERR_UNSUPPORTED before any launch, and the outputs stay untouched."""
    from nano_vllm_metal_amd import _lib

    lib = _lib.load()
    T = 2048
    size = ctypes.c_size_t()
    cap = ctypes.c_size_t()
    _lib.check(lib.nvm_moe_workspace_size(T, 2048, 768, 128, 8, ctypes.byref(size)))
    _lib.check(lib.nvm_moe_scratch_bytes(ctypes.byref(cap)))
    assert size.value > cap.value
    x, moe = _case(42, 8)
    xs = x.repeat(T // 8, 1).contiguous()
    head, flat, ops = _args(moe, xs)
    y = torch.full_like(xs, 3.0)
    rc = lib.nvm_moe_forward_noalloc(*head, *flat, y.data_ptr(), None, None, 0,
                                     _lib.stream_of(xs.device))
    torch.cuda.synchronize()
    assert rc == _lib.NVM_ERR_UNSUPPORTED
    assert b"static scratch" in lib.nvm_last_error()
    assert bool((y == 3.0).all())


def test_noalloc_call_captured_in_a_graph():
    """The entry point is for callers under HIP graph capture: one noalloc
    call captured in a torch CUDA graph (after nvm_moe_scratch_bytes located
    the array outside the capture), replayed three times with eager work and
    synchronisations between the replays, equals nvm_moe_forward bitwise on
    every replay."""
    from nano_vllm_metal_amd import _lib

    lib = _lib.load()
    cap = ctypes.c_size_t()
    _lib.check(lib.nvm_moe_scratch_bytes(ctypes.byref(cap)))
    x, moe = _case(43, 32)
    (y0, ids0, sc0), _, _ = _run_both(moe, x, 0)
    head, flat, ops = _args(moe, x)
    T, k = x.shape[0], moe.num_experts_per_tok
    y = torch.empty_like(x)
    ids = torch.empty((T, k), dtype=torch.int32, device=x.device)
    sc = torch.empty((T, k), dtype=x.dtype, device=x.device)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = lib.nvm_moe_forward_noalloc(*head, *flat, y.data_ptr(), ids.data_ptr(),
                                         sc.data_ptr(), 0, _lib.stream_of(x.device))
    assert rc == 0, lib.nvm_last_error()
    for rep in range(3):
        y.fill_(float("nan"))
        ids.fill_(-7)
        sc.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        print(f"noalloc graph replay {rep}", flush=True)
        for u, v, what in ((y0, y, "y"), (ids0, ids, "ids"), (sc0, sc, "scores")):
            assert torch.equal(u, v), f"replay {rep}: {what} differs from nvm_moe_forward"
    del ops
