"""MI355X-native Qwen3 sparse-MoE block with nano-vllm-metal's MoE interface.

Public names mirror the reference's package root for this path
(``src/nano_vllm_metal/__init__.py:6,8``): ``QuantizedWeights``,
``quantized_matmul``, ``quantized_linear``, ``route_topk``,
``grouped_expert_linear`` and ``Moe``, plus ``paged_attention``
(``layers/attention.py:154``), the Qwen3 model with its paged KV cache and
``LLM``/``SamplingParams`` (``llm.py``).  All compute runs in HIP kernels on the GPU
(libnvm_moe.so); nothing falls back to the CPU.
"""

from .linear import QuantizedWeights, dequantize, quantize, quantized_linear, quantized_matmul
from .moe import Moe, grouped_expert_linear, moe_dispatch, route_and_dispatch, route_topk
from .loader import load_moe_block, load_moe_blocks, read_config, sparse_layers
from .attention import paged_attention
from .kv_cache import PagedKVCache
from .qwen3 import Qwen3Config, Qwen3Model, qwen3_30b_a3b_config
from .llm import LLM, GenerationOutput, SamplingParams

__all__ = [
    "QuantizedWeights",
    "quantize",
    "dequantize",
    "quantized_matmul",
    "quantized_linear",
    "route_topk",
    "grouped_expert_linear",
    "moe_dispatch",
    "route_and_dispatch",
    "Moe",
    "load_moe_block",
    "load_moe_blocks",
    "read_config",
    "sparse_layers",
    "paged_attention",
    "PagedKVCache",
    "Qwen3Config",
    "Qwen3Model",
    "qwen3_30b_a3b_config",
    "LLM",
    "SamplingParams",
    "GenerationOutput",
]
