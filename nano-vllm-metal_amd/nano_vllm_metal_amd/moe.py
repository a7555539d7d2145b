"""The Qwen3 sparse-MoE block on MI355X.

Drop-in for layers/moe.py of nano-vllm-metal (paths relative to the
reference's ``src/nano_vllm_metal``): the same three names with the same
signatures and return shapes, on GPU torch tensors, computed by the HIP
kernels of libnvm_moe.so:

* ``route_topk(x, w_router, top_k, norm_topk_prob)`` (moe.py:37-49)
* ``grouped_expert_linear(x, w_experts, expert_ids)`` (moe.py:8-34)
* ``Moe(w_router, w_gate, w_up, w_down, num_experts_per_tok, norm_topk_prob)``
  and ``Moe.__call__(x)`` (moe.py:52-86)

plus ``moe_dispatch`` (the stable expert sort of moe.py:16-17, exposed so the
permutation itself can be checked).

Differences a caller can observe, all deliberate:

* ``route_topk`` returns ``uint32`` ids, as the reference's
  ``argpartition`` does; this module's own additions (``route_and_dispatch``,
  ``Moe.forward(..., return_routing=True)``) return ``int32`` ids, the same
  bits, since torch indexes with signed integers;
* top-k slots are in (probability desc, expert index asc) order; the
  reference's ``argpartition`` leaves slot order unspecified;
* the block is one call into the library (route, dispatch, fused gate/up +
  SwiGLU, down, combine) and does not materialise the k-fold copy of ``x``
  (moe.py:77-79).
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .linear import QuantizedWeights

REGIMES = {"auto": _lib.REGIME_AUTO, "decode": _lib.REGIME_DECODE,
           "prefill": _lib.REGIME_PREFILL}


def _i32(t: torch.Tensor) -> torch.Tensor:
    if t.dtype == torch.int32:
        return t.contiguous()
    if t.dtype == torch.uint32:
        return t.contiguous().view(torch.int32)
    return t.to(torch.int32).contiguous()


def _check_expert_weights(w: QuantizedWeights, act: torch.dtype, name: str) -> None:
    if w.scales.dtype != act or w.biases.dtype != act:
        raise ValueError(f"{name}: scales/biases must have the activation dtype {act}")
    if w.weight.dim() != 3:
        raise ValueError(f"{name}: expert weight must be [E, out, in/8]")


def _workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def route_topk(x: torch.Tensor, w_router: QuantizedWeights, top_k: int,
               norm_topk_prob: bool = False):
    """Router (moe.py:37-49) -> ``(probs [..., E], ids [..., k] uint32, scores [..., k])``.

    The ids are uint32, as ``mx.argpartition`` returns them (moe.py:45); the
    other entry points take them as they are (or as int32 / int64).
    """
    lib = _lib.load()
    dev = _lib.require_device(x, w_router.weight, w_router.scales, w_router.biases)
    *lead, H = x.shape
    x2 = x.reshape(-1, H).contiguous()
    T = x2.shape[0]
    E = w_router.weight.shape[0]
    wr = _i32(w_router.weight)
    probs = torch.empty((T, E), dtype=x.dtype, device=dev)
    ids = torch.empty((T, top_k), dtype=torch.uint32, device=dev)
    scores = torch.empty((T, top_k), dtype=x.dtype, device=dev)
    size = ctypes.c_size_t()
    _lib.check(lib.nvm_route_workspace_size(T, H, E, ctypes.byref(size)))
    ws = _workspace(size.value, dev)
    _lib.check(lib.nvm_moe_route(
        x2.data_ptr(), T, H, wr.data_ptr(), w_router.scales.contiguous().data_ptr(),
        w_router.biases.contiguous().data_ptr(), E, w_router.group_size, w_router.bits, top_k,
        int(bool(norm_topk_prob)), _lib.dtype_code(x.dtype), probs.data_ptr(), ids.data_ptr(),
        scores.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(dev)))
    return (probs.reshape(*lead, E), ids.reshape(*lead, top_k), scores.reshape(*lead, top_k))


def moe_dispatch(expert_ids: torch.Tensor, num_experts: int):
    """Stable sort of flat expert ids by expert (moe.py:16-17).

    Returns ``(offsets [E+1] int32, sorted_pairs [n] int32)``: ``sorted_pairs``
    lists flat indices into ``expert_ids`` grouped by expert in ascending
    order, ascending within an expert; ``offsets`` delimits the groups.
    """
    lib = _lib.load()
    dev = _lib.require_device(expert_ids)
    flat = _i32(expert_ids.reshape(-1))
    n = flat.numel()
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    sorted_pairs = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
    size = ctypes.c_size_t()
    _lib.check(lib.nvm_dispatch_workspace_size(n, num_experts, ctypes.byref(size)))
    ws = _workspace(size.value, dev)
    _lib.check(lib.nvm_moe_dispatch(flat.data_ptr(), n, num_experts, offsets.data_ptr(),
                                    sorted_pairs.data_ptr(), ws.data_ptr(), ws.numel(),
                                    _lib.stream_of(dev)))
    return offsets, sorted_pairs[:n]


def route_and_dispatch(x: torch.Tensor, w_router: QuantizedWeights, top_k: int,
                       norm_topk_prob: bool = False):
    """Routing then dispatch, the first stage of ``Moe`` (moe.py:37-49, 16-17).

    Returns ``(ids [T, k] int32, scores [T, k], offsets [E+1] int32,
    sorted_pairs [T*k] int32)`` for ``x`` of ``T`` tokens, as
    ``route_topk`` followed by ``moe_dispatch`` of the flat ids.
    """
    lib = _lib.load()
    dev = _lib.require_device(x, w_router.weight, w_router.scales, w_router.biases)
    H = x.shape[-1]
    x2 = x.reshape(-1, H).contiguous()
    T = x2.shape[0]
    E = w_router.weight.shape[0]
    ids = torch.empty((T, top_k), dtype=torch.int32, device=dev)
    scores = torch.empty((T, top_k), dtype=x.dtype, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    sorted_pairs = torch.empty(max(T * top_k, 1), dtype=torch.int32, device=dev)
    size = ctypes.c_size_t()
    _lib.check(lib.nvm_route_dispatch_workspace_size(T, H, E, top_k, ctypes.byref(size)))
    ws = _workspace(size.value, dev)
    _lib.check(lib.nvm_moe_route_dispatch(
        x2.data_ptr(), T, H, _i32(w_router.weight).data_ptr(),
        w_router.scales.contiguous().data_ptr(), w_router.biases.contiguous().data_ptr(), E,
        w_router.group_size, w_router.bits, top_k, int(bool(norm_topk_prob)),
        _lib.dtype_code(x.dtype), None, ids.data_ptr(), scores.data_ptr(), offsets.data_ptr(),
        sorted_pairs.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(dev)))
    return ids, scores, offsets, sorted_pairs[:T * top_k]


def grouped_expert_linear(x: torch.Tensor, w_experts: QuantizedWeights,
                          expert_ids: torch.Tensor, regime: str = "auto") -> torch.Tensor:
    """``out[r] = x[r] . dequant(W[expert_ids[r]])^T`` (moe.py:8-34).

    ``x`` is ``[..., D]`` and ``expert_ids`` has the shape of ``x[..., 0]``;
    returns ``[..., out_dim]``.  ``regime`` selects the decode GEMV or the
    prefill GEMM ("auto" picks by rows per expert).
    """
    lib = _lib.load()
    dev = _lib.require_device(x, expert_ids, w_experts.weight, w_experts.scales,
                              w_experts.biases)
    _check_expert_weights(w_experts, x.dtype, "grouped_expert_linear")
    *lead, D = x.shape
    x2 = x.reshape(-1, D).contiguous()
    ids = _i32(expert_ids.reshape(-1))
    if ids.numel() != x2.shape[0]:
        raise ValueError("expert_ids must have one id per row of x")
    E, O = w_experts.weight.shape[0], w_experts.weight.shape[1]
    n = x2.shape[0]
    out = torch.empty((n, O), dtype=x.dtype, device=dev)
    size = ctypes.c_size_t()
    _lib.check(lib.nvm_grouped_linear_workspace_size(n, D, O, E, ctypes.byref(size)))
    ws = _workspace(size.value, dev)
    _lib.check(lib.nvm_grouped_expert_linear(
        x2.data_ptr(), n, D, _i32(w_experts.weight).data_ptr(),
        w_experts.scales.contiguous().data_ptr(), w_experts.biases.contiguous().data_ptr(), E, O,
        w_experts.group_size, w_experts.bits, ids.data_ptr(), _lib.dtype_code(x.dtype),
        out.data_ptr(), REGIMES[regime], ws.data_ptr(), ws.numel(), _lib.stream_of(dev)))
    return out.reshape(*lead, O)


class Moe:
    """Qwen3 sparse-MoE block (moe.py:52-86) backed by one library call."""

    def __init__(self, w_router: QuantizedWeights, w_gate: QuantizedWeights,
                 w_up: QuantizedWeights, w_down: QuantizedWeights, num_experts_per_tok: int,
                 norm_topk_prob: bool = False):
        self.w_router = w_router
        self.w_gate = w_gate
        self.w_up = w_up
        self.w_down = w_down
        self.num_experts_per_tok = num_experts_per_tok
        self.norm_topk_prob = norm_topk_prob
        # the regime of the expert products; "auto" follows the routed batch size
        self.regime = "auto"
        self._ws = None
        self._retired_ws = []

    def _operands(self):
        return [(_i32(w.weight), w.scales.contiguous(), w.biases.contiguous())
                for w in (self.w_router, self.w_gate, self.w_up, self.w_down)]

    def _workspace(self, T: int, H: int, I: int, E: int, dev: torch.device) -> torch.Tensor:
        size = ctypes.c_size_t()
        lib = _lib.load()
        _lib.check(lib.nvm_moe_workspace_size(T, H, I, E, self.num_experts_per_tok,
                                              ctypes.byref(size)))
        if self._ws is None or self._ws.numel() < size.value or self._ws.device != dev:
            # A HIP graph captured earlier may still refer to the old buffer:
            # it stays alive with the block.  Replacements at least double
            # in size, so the retired buffers total less than the current one.
            need = size.value
            if self._ws is not None:
                if self._ws.device == dev:
                    need = max(need, 2 * self._ws.numel())
                self._retired_ws.append(self._ws)
            self._ws = _workspace(need, dev)
        return self._ws

    def check_operands(self, act: torch.dtype, H: int):
        """Validate the four weight sets against activations of dtype ``act``
        and hidden size ``H`` (the library takes one group size and bit width
        for all of them); returns ``(E, I)``."""
        for name, w in (("router", self.w_router), ("gate", self.w_gate), ("up", self.w_up),
                        ("down", self.w_down)):
            if w.scales.dtype != act or w.biases.dtype != act:
                raise ValueError(f"Moe: {name} scales/biases must have the activation dtype")
        gs = self.w_gate.group_size
        bits = self.w_gate.bits
        for w in (self.w_router, self.w_up, self.w_down):
            if w.group_size != gs or w.bits != bits:
                raise ValueError("Moe: all weights must share group_size and bits")
        E = self.w_router.weight.shape[0]
        I = self.w_gate.weight.shape[1]
        if self.w_router.weight.shape != (E, H // 8):
            raise ValueError("Moe: router weight must be [E, H/8]")
        if self.w_gate.weight.shape != (E, I, H // 8) or self.w_up.weight.shape != (E, I, H // 8):
            raise ValueError("Moe: gate/up weights must be [E, I, H/8]")
        if self.w_down.weight.shape != (E, H, I // 8):
            raise ValueError("Moe: down weight must be [E, H, I/8]")
        return E, I

    def forward(self, x: torch.Tensor, return_routing: bool = False):
        lib = _lib.load()
        dev = _lib.require_device(x, self.w_router.weight, self.w_gate.weight,
                                  self.w_up.weight, self.w_down.weight)
        *lead, H = x.shape
        E, I = self.check_operands(x.dtype, H)
        gs = self.w_gate.group_size
        bits = self.w_gate.bits
        x2 = x.reshape(-1, H).contiguous()
        T = x2.shape[0]
        k = self.num_experts_per_tok
        prep = self._operands()
        ws = self._workspace(T, H, I, E, dev)
        y = torch.empty_like(x2)
        ids = torch.empty((T, k), dtype=torch.int32, device=dev) if return_routing else None
        scores = torch.empty((T, k), dtype=x.dtype, device=dev) if return_routing else None
        (wr, sr, br), (wg, sg, bg), (wu, su, bu), (wd, sd, bd) = prep
        _lib.check(lib.nvm_moe_forward(
            x2.data_ptr(), T, H, I, E, k, int(bool(self.norm_topk_prob)), gs, bits,
            _lib.dtype_code(x.dtype),
            wr.data_ptr(), sr.data_ptr(), br.data_ptr(),
            wg.data_ptr(), sg.data_ptr(), bg.data_ptr(),
            wu.data_ptr(), su.data_ptr(), bu.data_ptr(),
            wd.data_ptr(), sd.data_ptr(), bd.data_ptr(),
            y.data_ptr(), _lib.ptr(ids), _lib.ptr(scores), REGIMES[self.regime],
            ws.data_ptr(), ws.numel(), _lib.stream_of(dev)))
        y = y.reshape(*lead, H)
        if return_routing:
            return y, ids.reshape(*lead, k), scores.reshape(*lead, k)
        return y

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        return self.forward(x)
