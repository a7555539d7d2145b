"""Local MLX-checkpoint loader (nano_vllm_metal_amd.loader).

Synthetic checkpoints in the MLX 4-bit layout are written to a temporary
directory (config.json plus safetensors, single-file and sharded) and read
back on the CPU; the GPU test runs a loaded block against the oracle.  The
sparse-layer rule follows models/qwen3.py:255-260 and the module wiring
models/qwen3.py:309-325.
"""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from helpers import assert_moe_close, to_act, to_np
from oracle import moe_oracle as O

H, I, E, K = 256, 128, 4, 2
DEV = "cuda:0"


def _t(a, act="bfloat16"):
    a = np.asarray(a)
    if a.dtype == np.uint32:
        return torch.from_numpy(a.copy())
    return torch.tensor(a, dtype=torch.bfloat16 if act == "bfloat16" else torch.float16)


def _layer_tensors(layer, w, per_expert=False):
    base = f"model.layers.{layer}.mlp"
    out = {}
    for field, arr in zip(("weight", "scales", "biases"), w["router"]):
        out[f"{base}.gate.{field}"] = _t(arr)
    for name, key in (("gate_proj", "gate"), ("up_proj", "up"), ("down_proj", "down")):
        for field, arr in zip(("weight", "scales", "biases"), w[key]):
            if per_expert:
                for j in range(arr.shape[0]):
                    out[f"{base}.experts.{j}.{name}.{field}"] = _t(arr[j])
            else:
                out[f"{base}.switch_mlp.{name}.{field}"] = _t(arr)
    return out


def _config(**over):
    cfg = {"num_hidden_layers": 4, "hidden_size": H, "moe_intermediate_size": I,
           "num_experts": E, "num_experts_per_tok": K, "norm_topk_prob": True,
           "decoder_sparse_step": 2, "mlp_only_layers": [3],
           "quantization": {"group_size": 64, "bits": 4}}
    cfg.update(over)
    return cfg


def _write(tmp_path, cfg, tensors, shards=1):
    from safetensors.torch import save_file

    (tmp_path / "config.json").write_text(json.dumps(cfg))
    names = sorted(tensors)
    if shards == 1:
        save_file(tensors, str(tmp_path / "model.safetensors"))
        return
    wmap = {}
    for s in range(shards):
        fn = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
        part = {n: tensors[n] for n in names[s::shards]}
        save_file(part, str(tmp_path / fn))
        wmap.update({n: fn for n in part})
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wmap}))


def _weights(seed=5):
    return O.make_inputs(seed, 8, H, E, I, "bfloat16")


def _same(qw, src, gs):
    wq, s, b = src
    assert qw.group_size == gs and qw.bits == 4
    assert qw.weight.dtype == torch.int32
    assert np.array_equal(qw.weight.view(torch.uint32).numpy(), wq)
    assert np.array_equal(qw.scales.float().numpy(), s)
    assert np.array_equal(qw.biases.float().numpy(), b)


def test_sparse_layers_rule():
    from nano_vllm_metal_amd import sparse_layers

    assert sparse_layers(_config()) == [1]
    assert sparse_layers(_config(decoder_sparse_step=1, mlp_only_layers=[])) == [0, 1, 2, 3]
    assert sparse_layers(_config(num_experts=0)) == []


@pytest.mark.parametrize("shards,per_expert", [(1, False), (3, False), (2, True)])
def test_load_block_matches_stored_tensors(tmp_path, shards, per_expert):
    from nano_vllm_metal_amd import load_moe_block, load_moe_blocks

    _, w = _weights()
    _write(tmp_path, _config(), _layer_tensors(1, w, per_expert), shards)
    moe = load_moe_block(tmp_path, 1, device="cpu")
    _same(moe.w_router, w["router"], 64)
    _same(moe.w_gate, w["gate"], 64)
    _same(moe.w_up, w["up"], 64)
    _same(moe.w_down, w["down"], 64)
    assert moe.num_experts_per_tok == K and moe.norm_topk_prob is True
    blocks = load_moe_blocks(tmp_path, device="cpu")
    assert list(blocks) == [1]


def test_per_module_quantization_override(tmp_path):
    from nano_vllm_metal_amd import load_moe_block

    rng = np.random.default_rng(3)
    _, w = _weights()
    w["router"] = O.quantize(O.round_act(rng.standard_normal((E, H)) * 0.02, "bfloat16"), 128, 4,
                             "bfloat16")
    q = {"group_size": 64, "bits": 4, "model.layers.1.mlp.gate": {"group_size": 128, "bits": 4}}
    _write(tmp_path, _config(quantization=q), _layer_tensors(1, w))
    moe = load_moe_block(tmp_path, 1, device="cpu")
    _same(moe.w_router, w["router"], 128)
    _same(moe.w_gate, w["gate"], 64)


def test_loader_rejects_what_the_kernels_cannot_run(tmp_path):
    from nano_vllm_metal_amd import load_moe_block

    _, w = _weights()
    tensors = _layer_tensors(1, w)
    _write(tmp_path, _config(quantization={"group_size": 64, "bits": 8}), tensors)
    with pytest.raises(ValueError, match="4-bit"):
        load_moe_block(tmp_path, 1, device="cpu")
    _write(tmp_path, _config(quantization={"group_size": 64, "bits": 4,
                                           "model.layers.1.mlp.gate": False}), tensors)
    with pytest.raises(ValueError, match="unquantised"):
        load_moe_block(tmp_path, 1, device="cpu")
    cfg = _config()
    del cfg["quantization"]
    _write(tmp_path, cfg, tensors)
    with pytest.raises(ValueError, match="quantization"):
        load_moe_block(tmp_path, 1, device="cpu")
    _write(tmp_path, _config(), tensors)
    with pytest.raises(ValueError, match="not a sparse"):
        load_moe_block(tmp_path, 0, device="cpu")
    del tensors["model.layers.1.mlp.switch_mlp.up_proj.weight"]
    _write(tmp_path, _config(), tensors)
    with pytest.raises(KeyError):
        load_moe_block(tmp_path, 1, device="cpu")


@pytest.mark.gpu
def test_loaded_block_matches_oracle(tmp_path):
    """A block read from a sharded checkpoint runs on the GPU to the oracle's
    routing (exact) and outputs (tolerance)."""
    from nano_vllm_metal_amd import load_moe_block

    x, w = _weights(9)
    _write(tmp_path, _config(), _layer_tensors(1, w), shards=2)
    moe = load_moe_block(tmp_path, 1, device=DEV)
    y, ids, scores = moe.forward(to_act(x, "bfloat16", DEV), return_routing=True)
    torch.cuda.synchronize()
    y_ref, ids_ref, sc_ref = O.moe_forward(x, w, K, True, "bfloat16", 64)
    assert np.array_equal(ids.cpu().numpy(), ids_ref)
    assert np.array_equal(to_np(scores), sc_ref)
    assert_moe_close(y, y_ref, "bfloat16", "loaded block")
