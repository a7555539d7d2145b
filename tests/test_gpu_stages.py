"""nvm_moe_forward_stage: the block's launch sequence one stage at a time.

Stages 0..3 (and 0, 4, 5: both products as the forward launches them, then
their combine) run in order on one workspace must give exactly what
nvm_moe_forward gives (the same kernels, the same workspace hand-offs), for
each of the launch sequences the forward takes: decode batches (routing
finalised in the gate/up prologue; both products in one launch from 32
tokens), prefill batches whose int8 router writes the fp16 copy of x,
prefill batches converted by their own launch, and fp16 activations.
Repeating a stage must not change what the next one reads.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from helpers import make_moe, to_act
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _call(lib, L, moe, x, ws, y, ids, sc, stage=None, regime=0):
    T, H = x.shape
    E, I = moe.check_operands(x.dtype, H)
    ops = moe._operands()
    flat = [t.data_ptr() for trio in ops for t in trio]
    head = [x.data_ptr(), T, H, I, E, moe.num_experts_per_tok, int(moe.norm_topk_prob),
            moe.w_gate.group_size, moe.w_gate.bits, L.dtype_code(x.dtype)]
    tail = [y.data_ptr(), ids.data_ptr(), sc.data_ptr(), regime, ws.data_ptr(), ws.numel(),
            L.stream_of(x.device)]
    if stage is None:
        L.check(lib.nvm_moe_forward(*head, *flat, *tail))
    else:
        L.check(lib.nvm_moe_forward_stage(stage, *head, *flat, *tail))
    torch.cuda.synchronize()


@pytest.mark.parametrize("T,act,regime,seq", [
    (32, "bfloat16", 0, (0, 1, 2, 3)),  # decode: partial logits, gate/up finalising the routing
    (300, "bfloat16", 0, (0, 1, 2, 3)),  # prefill: int8 router writes the fp16 copy of x
    (100, "bfloat16", 2, (0, 1, 2, 3)),  # prefill below the int8 router's batch: act_to_f16
    (200, "float16", 0, (0, 1, 2, 3)),  # fp16 activations: the GEMMs stage x themselves
    (32, "bfloat16", 0, (0, 4, 5)),     # decode, both products in one launch, split combine
    (64, "float16", 0, (0, 4, 5)),
    (8, "bfloat16", 0, (0, 4, 5)),      # stage 4 as stages 1 and 2 (no fused launch)
])
def test_stages_in_order_equal_the_forward(T, act, regime, seq):
    from nano_vllm_metal_amd import _lib as L

    lib = L.load()
    x, w = O.make_packed_inputs(7 + T, T, 2048, 128, 768, act, 64)
    x = to_act(x, act, DEV)
    moe = make_moe(w, act, 64, 8, True, DEV)
    k = moe.num_experts_per_tok
    size = ctypes.c_size_t()
    L.check(lib.nvm_moe_workspace_size(T, 2048, 768, 128, k, ctypes.byref(size)))
    outs = []
    for staged in (False, True):
        ws = torch.empty(size.value, dtype=torch.uint8, device=DEV)
        y = torch.full_like(x, float("nan"))
        ids = torch.full((T, k), -1, dtype=torch.int32, device=DEV)
        sc = torch.full((T, k), float("nan"), dtype=x.dtype, device=DEV)
        if staged:
            for s in seq:
                # every stage twice: a repeat must leave the next stage's inputs as they were
                for _ in range(2):
                    _call(lib, L, moe, x, ws, y, ids, sc, stage=s, regime=regime)
        else:
            _call(lib, L, moe, x, ws, y, ids, sc, regime=regime)
        outs.append((y, ids, sc))
    print(f"stages T={T} {act} regime={regime} seq={seq}", flush=True)
    for a, b, what in zip(outs[0], outs[1], ("y", "ids", "scores")):
        assert torch.equal(a, b), f"{what} of the staged calls differs from nvm_moe_forward"


@pytest.mark.parametrize("T", [4096, 300, 129])
def test_prefill_gemm_with_direct_to_lds_staging_is_bit_identical(T, monkeypatch):
    """The forward's GEMMs on their fp16 copies stage activations straight
    into LDS (gemm_dma_kernel); NVM_GEMM_NODMA=1 takes the register-staged
    kernel of the same arithmetic.  Both must give the same bits: 4096
    tokens (the headline prefill), 300 (ragged m-tiles) and 129 (one more
    than the int8 router's threshold, many short tiles); the down product's
    12 k-steps end in a partial trip of the k-loop."""
    from nano_vllm_metal_amd import _lib as L

    lib = L.load()
    x, w = O.make_packed_inputs(800 + T, T, 2048, 128, 768, "bfloat16", 64)
    x = to_act(x, "bfloat16", DEV)
    moe = make_moe(w, "bfloat16", 64, 8, True, DEV)
    moe.regime = "prefill"
    outs = []
    for nodma in ("1", "0"):
        monkeypatch.setenv("NVM_GEMM_NODMA", nodma)
        y, ids, sc = moe.forward(x, return_routing=True)
        torch.cuda.synchronize()
        outs.append((y.clone(), ids.clone(), sc.clone()))
    print(f"dma vs register staging T={T}", flush=True)
    for a, b, what in zip(outs[0], outs[1], ("y", "ids", "scores")):
        assert torch.equal(a, b), f"{what}: direct-to-LDS GEMM differs from register staging"
