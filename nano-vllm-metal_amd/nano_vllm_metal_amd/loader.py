"""Local-path loader for the MoE blocks of an MLX 4-bit Qwen3-MoE checkpoint.

The reference builds its blocks from a model loaded by ``mlx_lm.load``
(``models/qwen3.py:296-325``, ``loader.py:30-36``): for each sparse layer
``mlp.gate`` is the router and ``mlp.switch_mlp.{gate,up,down}_proj`` are the
stacked expert projections, each an MLX ``QuantizedLinear`` /
``QuantizedSwitchLinear`` whose ``weight``, ``scales``, ``biases``,
``group_size`` and ``bits`` go into ``QuantizedWeights``
(``layers/linear.py:62-70``).  Which layers are sparse follows
``is_qwen3_moe_sparse_layer`` (``models/qwen3.py:255-260``).

This module reads the same tensors straight from a local checkpoint directory
(``config.json`` plus ``model.safetensors`` or a sharded
``model.safetensors.index.json``), with no hub access:

* ``quantization`` in ``config.json`` gives the default ``group_size`` and
  ``bits``; an entry keyed by a module path (for example
  ``"model.layers.3.mlp.gate"``) overrides them for that module, and ``false``
  there marks it unquantised (not supported: the kernels take 4-bit weights).
* Expert projections stored per expert (``mlp.experts.{j}.gate_proj.*``, the
  layout before MLX stacks them) are stacked along a new leading axis, so they
  land in the same ``[E, out, in/8]`` layout as ``switch_mlp``.

Tensors keep the MLX layout (no repacking): ``weight`` as int32 bit patterns
of the uint32 words, ``scales``/``biases`` in the activation dtype.  Loading
uses safetensors' own reader, which executes nothing from the file.
"""

from __future__ import annotations

import json
from pathlib import Path
from typing import Dict, Iterable, List, Optional

import torch

from .linear import QuantizedWeights
from .moe import Moe

_PROJS = ("gate_proj", "up_proj", "down_proj")


def read_config(path) -> dict:
    """``config.json`` of the checkpoint directory."""
    with open(Path(path) / "config.json") as f:
        return json.load(f)


def sparse_layers(config: dict) -> List[int]:
    """Layer indices whose MLP is the sparse-MoE block
    (``is_qwen3_moe_sparse_layer``, ``models/qwen3.py:255-260``)."""
    n = int(config["num_hidden_layers"])
    if int(config.get("num_experts", 0)) <= 0:
        return []
    only = set(config.get("mlp_only_layers", []) or [])
    step = int(config.get("decoder_sparse_step", 1) or 1)
    return [i for i in range(n) if i not in only and (i + 1) % step == 0]


def quant_params(config: dict, module: str):
    """``(group_size, bits)`` of a module: the per-module entry of
    ``quantization`` if there is one, else the checkpoint default."""
    q = config.get("quantization", config.get("quantization_config"))
    if not isinstance(q, dict):
        raise ValueError("checkpoint has no 'quantization' entry: not an MLX quantised model")
    own = q.get(module, None)
    if own is False:
        raise ValueError(f"{module} is stored unquantised; the MoE kernels take 4-bit weights")
    src = own if isinstance(own, dict) else q
    if "group_size" not in src or "bits" not in src:
        raise ValueError(f"no group_size/bits for {module} in 'quantization'")
    return int(src["group_size"]), int(src["bits"])


class _Tensors:
    """Lazy name -> tensor access over one or several safetensors files."""

    def __init__(self, path: Path):
        from safetensors import safe_open

        index = path / "model.safetensors.index.json"
        if index.exists():
            with open(index) as f:
                wmap = json.load(f)["weight_map"]
            files = sorted(set(wmap.values()))
        else:
            single = path / "model.safetensors"
            if not single.exists():
                raise FileNotFoundError(f"no model.safetensors or index in {path}")
            files = [single.name]
            wmap = None
        self._handles = {fn: safe_open(str(path / fn), framework="pt") for fn in files}
        if wmap is None:
            wmap = {k: files[0] for k in self._handles[files[0]].keys()}
        self._where = wmap

    def has(self, name: str) -> bool:
        return name in self._where

    def get(self, name: str) -> torch.Tensor:
        if name not in self._where:
            raise KeyError(f"tensor {name!r} not in the checkpoint")
        return self._handles[self._where[name]].get_tensor(name)

    def names(self) -> Iterable[str]:
        return self._where.keys()


def _words(t: torch.Tensor) -> torch.Tensor:
    """uint32 words as int32 bit patterns (the carrier's weight dtype)."""
    if t.dtype == torch.int32:
        return t
    if t.dtype == torch.uint32:
        return t.view(torch.int32)
    raise ValueError(f"packed weights must be uint32, got {t.dtype}")


def _qweights(ts: _Tensors, prefix: str, config: dict, device, stack: Optional[int] = None):
    gs, bits = quant_params(config, prefix if stack is None else prefix.replace("{j}", "0"))
    if bits != 4:
        raise ValueError(f"{prefix}: {bits}-bit weights; the MoE kernels take 4-bit weights")

    def fetch(field):
        if stack is None:
            return ts.get(f"{prefix}.{field}")
        return torch.stack([ts.get(f"{prefix.format(j=j)}.{field}") for j in range(stack)])

    w, s, b = _words(fetch("weight")), fetch("scales"), fetch("biases")
    if s.shape != b.shape or s.shape[:-1] != w.shape[:-1]:
        raise ValueError(f"{prefix}: inconsistent shapes {tuple(w.shape)}, {tuple(s.shape)}, "
                         f"{tuple(b.shape)}")
    if w.shape[-1] * (32 // bits) != s.shape[-1] * gs:
        raise ValueError(f"{prefix}: weight and scales disagree with group_size {gs}")
    return QuantizedWeights(s.contiguous().to(device), b.contiguous().to(device), gs, bits,
                            w.contiguous().to(device))


def load_moe_block(path, layer: int, device="cuda", config: Optional[dict] = None,
                   tensors: Optional[_Tensors] = None) -> Moe:
    """The ``Moe`` of sparse layer ``layer`` (``models/qwen3.py:309-325``)."""
    path = Path(path)
    config = read_config(path) if config is None else config
    if layer not in sparse_layers(config):
        raise ValueError(f"layer {layer} is not a sparse-MoE layer of this checkpoint")
    ts = _Tensors(path) if tensors is None else tensors
    base = f"model.layers.{layer}.mlp"
    router = _qweights(ts, f"{base}.gate", config, device)
    E = int(config["num_experts"])
    projs = {}
    for p in _PROJS:
        if ts.has(f"{base}.switch_mlp.{p}.weight"):
            projs[p] = _qweights(ts, f"{base}.switch_mlp.{p}", config, device)
        elif ts.has(f"{base}.experts.0.{p}.weight"):
            projs[p] = _qweights(ts, f"{base}.experts.{{j}}.{p}", config, device, stack=E)
        else:
            raise KeyError(f"no {base}.switch_mlp.{p} or {base}.experts.*.{p} in the checkpoint")
    if router.weight.shape[0] != E or projs["gate_proj"].weight.shape[0] != E:
        raise ValueError(f"layer {layer}: expert count differs from num_experts={E}")
    return Moe(router, projs["gate_proj"], projs["up_proj"], projs["down_proj"],
               num_experts_per_tok=int(config["num_experts_per_tok"]),
               norm_topk_prob=bool(config.get("norm_topk_prob", False)))


def load_moe_blocks(path, device="cuda", layers: Optional[Iterable[int]] = None) -> Dict[int, Moe]:
    """Every sparse-MoE block of the checkpoint (or those of ``layers``)."""
    path = Path(path)
    config = read_config(path)
    ts = _Tensors(path)
    wanted = sparse_layers(config) if layers is None else list(layers)
    return {i: load_moe_block(path, i, device, config, ts) for i in wanted}
