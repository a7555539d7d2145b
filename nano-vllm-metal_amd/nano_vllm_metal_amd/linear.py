"""Quantised weight carrier and the dense W4A16 matmul.

Mirrors layers/linear.py of nano-vllm-metal (reference paths relative to
``src/nano_vllm_metal``): ``QuantizedWeights`` (linear.py:47-70),
``quantized_matmul`` (linear.py:73-89 -> metal/bindings.cpp:16-32) and
``quantized_linear`` (linear.py:92-126), on torch tensors resident on the GPU.

The MLX affine int4 layout is kept as is (no repacking at load time):
``weight`` uint32 ``[..., out, in/8]`` with code j of each word in bits
[4j, 4j+4), ``scales``/``biases`` in the activation dtype ``[..., out, in/group]``,
``w = q * scale + bias``.

``quantize``/``dequantize`` restate MLX's ``mx.quantize``/``mx.dequantize`` in
torch so that synthetic weights can be produced directly on the device (the
reference obtains its weights from MLX); they are layout utilities, not part of
the MoE hot path.
"""

from __future__ import annotations

from typing import Any

import torch

from . import _lib


class QuantizedWeights:
    """The five fields of the reference's ``QuantizedWeights`` (linear.py:47-60)."""

    def __init__(self, scales: torch.Tensor, biases: torch.Tensor, group_size: int, bits: int,
                 weight: torch.Tensor):
        self.scales = scales
        self.biases = biases
        self.group_size = group_size
        self.bits = bits
        self.weight = weight

    @staticmethod
    def from_mlx_layer(layer: Any) -> "QuantizedWeights":
        """Wrap any object with ``scales/biases/group_size/bits/weight`` fields
        (linear.py:62-70); the tensors are referenced, not copied."""
        return QuantizedWeights(scales=layer.scales, biases=layer.biases,
                                group_size=layer.group_size, bits=layer.bits,
                                weight=layer.weight)

    @property
    def in_features(self) -> int:
        return self.weight.shape[-1] * (32 // self.bits)

    @property
    def out_features(self) -> int:
        return self.weight.shape[-2]

    def to(self, device) -> "QuantizedWeights":
        return QuantizedWeights(self.scales.to(device), self.biases.to(device), self.group_size,
                                self.bits, self.weight.to(device))


def _u32_view_as_i32(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.int32 else t.view(torch.int32)


def quantize(w: torch.Tensor, group_size: int = 64, bits: int = 4):
    """MLX affine quantisation of ``w[..., n]`` -> ``(wq, scales, biases)``.

    Restates MLX 0.29's affine quantizer: per group the larger-magnitude edge
    is kept exact, the scale is signed so codes stay in [0, 15] and is
    adjusted so zero is representable.  Scales/biases take ``w.dtype``; codes
    are computed against the rounded scale/bias.  ``wq`` is int32 holding the
    uint32 bit patterns (torch has no full uint32 support).
    """
    if bits != 4:
        raise ValueError("only 4-bit quantisation is supported")
    n = w.shape[-1]
    if n % group_size:
        raise ValueError(f"last dim {n} not divisible by group_size {group_size}")
    act = w.dtype
    g = w.float().reshape(*w.shape[:-1], n // group_size, group_size)
    n_bins = float((1 << bits) - 1)
    w_max = g.amax(dim=-1)
    w_min = g.amin(dim=-1)
    mask = w_min.abs() > w_max.abs()
    scales = torch.clamp((w_max - w_min) / n_bins, min=1e-7)
    scales = torch.where(mask, scales, -scales)
    edge = torch.where(mask, w_min, w_max)
    q0 = torch.round(edge / scales)
    nz = q0 != 0
    scales = torch.where(nz, edge / torch.where(nz, q0, torch.ones_like(q0)), scales)
    biases = torch.where(nz, edge, torch.zeros_like(edge))
    scales = scales.to(act)
    scales = torch.where(scales == 0, torch.full_like(scales, 1e-7), scales)
    biases = biases.to(act)
    q = torch.round((g - biases.float()[..., None]) / scales.float()[..., None])
    q = q.clamp_(0, n_bins).to(torch.int64).reshape(*w.shape[:-1], n // 8, 8)
    shifts = torch.arange(0, 32, 4, device=w.device, dtype=torch.int64)
    wq = (q << shifts).sum(dim=-1)
    wq = torch.where(wq >= 2 ** 31, wq - 2 ** 32, wq).to(torch.int32)
    return wq, scales, biases


def dequantize(wq: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, group_size: int,
               bits: int = 4) -> torch.Tensor:
    """``q * scale + bias`` in float32 (exact), shape ``[..., in]``."""
    if bits != 4:
        raise ValueError("only 4-bit quantisation is supported")
    w = _u32_view_as_i32(wq).to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(0, 32, 4, device=w.device, dtype=torch.int64)
    q = ((w[..., None] >> shifts) & 0xF).reshape(*w.shape[:-1], w.shape[-1] * 8).float()
    n = q.shape[-1]
    qg = q.reshape(*q.shape[:-1], n // group_size, group_size)
    out = qg * scales.float()[..., None] + biases.float()[..., None]
    return out.reshape(q.shape)


def quantized_matmul(scales: torch.Tensor, biases: torch.Tensor, group_size: int, bits: int,
                     a: torch.Tensor, b: torch.Tensor, transpose_b: bool = False) -> torch.Tensor:
    """``a[..., N] . dequant(b[K, N/8])^T -> [..., K]`` on the GPU.

    Mirrors linear.py:73-89 / ``_ext.quantized_matmul``: ``transpose_b`` must
    be True (quantized_matmul.cpp:56-58), ``a``, ``scales`` and ``biases`` share
    the f16/bf16 dtype (:26-37).  Router-sized products (up to 512 outputs
    over up to 64 rows) accumulate in float64 and round once to ``a.dtype``;
    the rest run on the expert GEMV or GEMM as a single expert, accumulating
    in float32 like the reference's kernels (quantized_matmul.metal:25-44).
    """
    lib = _lib.load()
    if a.dtype != scales.dtype or scales.dtype != biases.dtype:
        raise ValueError("quantized_matmul: a, scales and biases must share a dtype")
    dev = _lib.require_device(a, b, scales, biases)
    *lead, N = a.shape
    a2 = a.reshape(-1, N).contiguous()
    b = _u32_view_as_i32(b).contiguous()
    scales = scales.contiguous()
    biases = biases.contiguous()
    if b.dim() != 2:
        raise ValueError("quantized_matmul: b must be 2-D")
    K = b.shape[0]
    if b.shape[1] * 8 != N or scales.shape != (K, N // group_size) or biases.shape != scales.shape:
        raise ValueError("quantized_matmul: shapes of a, b, scales, biases do not agree")
    out = torch.empty((a2.shape[0], K), dtype=a.dtype, device=dev)
    _lib.check(lib.nvm_quantized_matmul(
        scales.data_ptr(), biases.data_ptr(), group_size, bits, a2.data_ptr(), b.data_ptr(),
        int(bool(transpose_b)), out.data_ptr(), a2.shape[0], N, K, _lib.dtype_code(a.dtype),
        _lib.stream_of(dev)))
    return out.reshape(*lead, K)


def quantized_linear(x: torch.Tensor, w: QuantizedWeights,
                     bias: torch.Tensor | None = None) -> torch.Tensor:
    """``x . dequant(w)^T (+ bias)`` (linear.py:92-126) through the HIP matmul."""
    out = quantized_matmul(w.scales, w.biases, w.group_size, w.bits, x, w.weight, True)
    if bias is not None:
        out = out + bias
    return out
