"""Qwen3 / Qwen3-MoE forward on the MI355X kernels, with a paged KV cache.

A torch port of the reference's ``Qwen3PagedModel`` (``models/qwen3.py``):

* attention (``:18-173``): q/k/v through ``quantized_linear``, per-head
  RMSNorm of q and k, RoPE (``layers/rotary_embedding.py``, non-traditional
  half split, float32 tables), the new k/v written to the layer's page pool,
  then float32 attention: dense causal SDPA for a batch that starts from an
  empty cache (``:134-141``), ``paged_attention`` otherwise (``:150-161``);
* the block (``:186-252``): pre-norm residual attention and MLP, the MLP
  being ``Moe`` on sparse layers (``is_qwen3_moe_sparse_layer``,
  ``:255-260``) and the dense SwiGLU MLP elsewhere (``:176-184``);
* the model (``:263-394``): quantised embedding (``layers/embed_head.py``),
  final RMSNorm, lm head (or the tied embedding as a linear).

Every step runs on this package's HIP kernels: the q/k/v projections as one
``quantized_linear`` over stacked weights, per-head norm + RoPE + k/v store
in one kernel, ``paged_attention``, ``Moe``, and the residual adds fused with
the RMSNorm that follows each.  The initial prefill's causal attention over
the new tokens is torch's SDPA (float32, as the reference's
``mx.fast.scaled_dot_product_attention``).  Activations are bf16 (or fp16)
like the reference's ``precision``; norms and RoPE compute in float32 and
round where the reference materialises a tensor.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from pathlib import Path
from typing import List, Optional, Sequence

import torch

from .attention import causal_attention, causal_attention_supports, paged_attention
from .fused import embedding, moe_residual_rms_norm, qk_norm_rope_store, residual_rms_norm
from .kv_cache import PagedKVCache
from .linear import QuantizedWeights, quantized_linear
from .moe import Moe


@dataclass
class Qwen3Config:
    """The ``config.json`` fields the model reads (mlx_lm's ModelArgs)."""

    hidden_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    vocab_size: int
    head_dim: int = 0
    intermediate_size: int = 0
    moe_intermediate_size: int = 0
    num_experts: int = 0
    num_experts_per_tok: int = 0
    norm_topk_prob: bool = False
    decoder_sparse_step: int = 1
    mlp_only_layers: List[int] = field(default_factory=list)
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1000000.0
    max_position_embeddings: int = 32768
    tie_word_embeddings: bool = False

    @classmethod
    def from_dict(cls, d: dict) -> "Qwen3Config":
        names = cls.__dataclass_fields__.keys()
        cfg = cls(**{k: d[k] for k in names if k in d and d[k] is not None})
        if not cfg.head_dim:
            cfg.head_dim = cfg.hidden_size // cfg.num_attention_heads
        return cfg

    def is_sparse(self, layer: int) -> bool:
        """``is_qwen3_moe_sparse_layer`` (models/qwen3.py:255-260)."""
        return (self.num_experts > 0 and layer not in (self.mlp_only_layers or [])
                and (layer + 1) % (self.decoder_sparse_step or 1) == 0)


class RoPE:
    """The float32 cos/sin tables of ``layers/rotary_embedding.py:RoPE``
    (``traditional=False``): angle ``position * base ** (-i / (D/2))``; the
    rotation itself runs in the fused q/k kernel."""

    def __init__(self, dims: int, max_positions: int, base: float, device):
        half = dims // 2
        inv = torch.pow(torch.tensor(float(base), dtype=torch.float32),
                        -(torch.arange(half, dtype=torch.float32) / half))
        freqs = torch.outer(torch.arange(max_positions, dtype=torch.float32), inv)
        self.cos = torch.cos(freqs).to(device).contiguous()
        self.sin = torch.sin(freqs).to(device).contiguous()


class DenseMLP:
    """``Qwen3MLP`` (models/qwen3.py:176-184): down(silu(gate(x)) * up(x))."""

    def __init__(self, w_gate: QuantizedWeights, w_up: QuantizedWeights, w_down: QuantizedWeights):
        self.w_gate, self.w_up, self.w_down = w_gate, w_up, w_down

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        g = quantized_linear(x, self.w_gate)
        u = quantized_linear(x, self.w_up)
        return quantized_linear(silu(g) * u, self.w_down)


def silu(x: torch.Tensor) -> torch.Tensor:
    """``silu`` of layers/activation.py:21-24 as the same element-wise ops on
    tensors of the activation dtype, each result rounded to that dtype."""
    sig = 1 / (1 + torch.exp(-torch.abs(x)))
    sig = torch.where(x < 0, 1 - sig, sig)
    return x * sig


@dataclass
class StepInputs:
    """Device index tensors of one model step (see ``Qwen3Model.prepare``)."""

    positions: torch.Tensor    # [B*L] int32: position of each new token
    page_ids: torch.Tensor     # [B*L] int32: its page
    slots: torch.Tensor        # [B*L] int32: its slot in the page
    block_table: torch.Tensor  # [B, max_pages] int32
    lens: torch.Tensor         # [B] int32: context length after the step
    initial: bool              # every request starts from an empty cache


@dataclass
class Qwen3Layer:
    wq: QuantizedWeights
    wk: QuantizedWeights
    wv: QuantizedWeights
    wo: QuantizedWeights
    q_norm: torch.Tensor
    k_norm: torch.Tensor
    input_norm: torch.Tensor
    post_norm: torch.Tensor
    mlp: object  # Moe or DenseMLP
    wqkv: Optional[QuantizedWeights] = None  # q, k and v stacked along the output rows


def stack_outputs(*ws: QuantizedWeights) -> QuantizedWeights:
    """One product for several projections of the same input: rows, scales
    and biases concatenated along the output dimension."""
    gs, bits = ws[0].group_size, ws[0].bits
    if any(w.group_size != gs or w.bits != bits for w in ws):
        raise ValueError("stack_outputs: projections differ in group_size or bits")
    return QuantizedWeights(torch.cat([w.scales for w in ws]), torch.cat([w.biases for w in ws]),
                            gs, bits, torch.cat([w.weight for w in ws]))


class Qwen3Model:
    def __init__(self, config: Qwen3Config, embed: QuantizedWeights, layers: Sequence[Qwen3Layer],
                 norm: torch.Tensor, lm_head: Optional[QuantizedWeights],
                 dtype: torch.dtype = torch.bfloat16):
        self.config = config
        self.embed_w = embed
        self.layers = list(layers)
        self.norm = norm
        self.lm_head = lm_head
        self.dtype = dtype
        self.device = embed.weight.device
        self.rope = RoPE(config.head_dim, config.max_position_embeddings, config.rope_theta,
                         self.device)
        for layer in self.layers:
            if layer.wqkv is None:
                layer.wqkv = stack_outputs(layer.wq, layer.wk, layer.wv)

    # ---------------------------------------------------------------- pieces

    def create_kv_cache(self, num_pages: int, page_size: int = 16) -> PagedKVCache:
        c = self.config
        return PagedKVCache(c.num_hidden_layers, c.num_key_value_heads, c.head_dim, num_pages,
                            page_size, self.dtype, self.device)

    def embed(self, tokens: torch.Tensor) -> torch.Tensor:
        """``QuantizedEmbedding`` (layers/embed_head.py:21-36): dequantised rows
        (``nvm_embedding``)."""
        # (mx.dequantize returns the scales' dtype; a table stored in another
        # dtype than the model's is then cast, as the reference's next op does)
        w = self.embed_w
        return embedding(tokens, w, w.scales.dtype).to(self.dtype)

    def _attention(self, li: int, layer: Qwen3Layer, x: torch.Tensor, step: "StepInputs",
                   cache: PagedKVCache) -> torch.Tensor:
        c = self.config
        B, L, _ = x.shape
        Hq, Hkv, D = c.num_attention_heads, c.num_key_value_heads, c.head_dim
        qkv = quantized_linear(x, layer.wqkv)
        q, k, v = qk_norm_rope_store(qkv, Hq, Hkv, D, layer.q_norm, layer.k_norm, c.rms_norm_eps,
                                     step.positions, self.rope.cos, self.rope.sin, step.page_ids,
                                     step.slots, cache.key_pages[li], cache.value_pages[li],
                                     want_kv=step.initial)
        scale = D ** -0.5
        if step.initial and causal_attention_supports(Hq, Hkv, D):
            # every request starts from an empty cache: causal attention over
            # the new tokens only (models/qwen3.py:134-141); the grouped query
            # heads share each key/value read
            o = causal_attention(q.view(B, L, Hq, D), k.view(B, L, Hkv, D), v.view(B, L, Hkv, D),
                                 scale, self.dtype, out_dtype=x.dtype)
            o = o.reshape(B, L, Hq * D)
        else:
            # (the k/v of an initial step are in the pages as well)
            o = paged_attention(q.view(B, L, Hq, D).transpose(1, 2), cache.key_pages[li],
                                cache.value_pages[li], step.block_table, step.lens,
                                cache.page_size, scale=scale, mask="causal", out_dtype=x.dtype)
            o = o.transpose(1, 2).reshape(B, L, Hq * D)
        return quantized_linear(o, layer.wo)

    # ---------------------------------------------------------------- forward

    def prepare(self, cache: PagedKVCache, seq_ids: Sequence[int], L: int,
                width: Optional[int] = None) -> "StepInputs":
        """Host bookkeeping of one step: reserve pages for the next L tokens of
        every request and build the step's index tensors."""
        starts = [cache.lens[s] for s in seq_ids]
        for s in seq_ids:
            cache.reserve(s, L)
        page_ids, slots = cache.slot_mapping(seq_ids, L)
        block_table, lens = cache.block_table(seq_ids, extra=L, width=width)
        positions = torch.tensor([st + j for st in starts for j in range(L)], dtype=torch.int32,
                                 device=self.device)
        return StepInputs(positions, page_ids, slots, block_table, lens,
                          L > 1 and all(st == 0 for st in starts))

    def run(self, tokens: torch.Tensor, step: "StepInputs", cache: PagedKVCache,
            last_only: bool = True) -> torch.Tensor:
        """The device work of one step (no host synchronisation: it can be
        captured in a HIP graph)."""
        eps = self.config.rms_norm_eps
        h = self.embed(tokens)
        # residual adds fused with the norm that follows them
        _, x = residual_rms_norm(h, None, self.layers[0].input_norm, eps)
        n = len(self.layers)
        for li, layer in enumerate(self.layers):
            h, x = residual_rms_norm(h, self._attention(li, layer, x, step, cache),
                                     layer.post_norm, eps)
            nxt = self.layers[li + 1].input_norm if li + 1 < n else self.norm
            if isinstance(layer.mlp, Moe):
                # the MoE combine fused into this residual add and norm
                h, x = moe_residual_rms_norm(layer.mlp, x, h, nxt, eps)
            else:
                h, x = residual_rms_norm(h, layer.mlp(x), nxt, eps)
        if last_only:
            x = x[:, -1]
        return quantized_linear(x, self.lm_head if self.lm_head is not None else self.embed_w)

    def forward(self, tokens: torch.Tensor, cache: PagedKVCache, seq_ids: Sequence[int],
                last_only: bool = True) -> torch.Tensor:
        """Run ``tokens [B, L]`` (the next L tokens of each request) through the
        model, appending their keys/values to ``cache``.  Returns the logits of
        the last position ``[B, vocab]`` or of every position ``[B, L, vocab]``."""
        B, L = tokens.shape
        if len(seq_ids) != B:
            raise ValueError("forward: one sequence id per batch row")
        step = self.prepare(cache, seq_ids, L)
        logits = self.run(tokens.to(self.device), step, cache, last_only)
        cache.advance(seq_ids, L)
        return logits

    __call__ = forward

    # ---------------------------------------------------------------- builders

    @classmethod
    def from_checkpoint(cls, path, device="cuda", dtype: torch.dtype = torch.bfloat16):
        """Load an MLX 4-bit Qwen3 / Qwen3-MoE checkpoint from a local directory
        (``config.json`` plus safetensors, sharded or not)."""
        from .loader import _Tensors, _qweights, load_moe_block, read_config

        path = Path(path)
        raw = read_config(path)
        cfg = Qwen3Config.from_dict(raw)
        ts = _Tensors(path)

        def vec(name):
            return ts.get(name).to(device=device, dtype=dtype)

        layers = []
        for i in range(cfg.num_hidden_layers):
            base = f"model.layers.{i}"
            att = f"{base}.self_attn"
            if cfg.is_sparse(i):
                mlp = load_moe_block(path, i, device, raw, ts)
            else:
                mlp = DenseMLP(*[_qweights(ts, f"{base}.mlp.{p}", raw, device)
                                 for p in ("gate_proj", "up_proj", "down_proj")])
            layers.append(Qwen3Layer(
                *[_qweights(ts, f"{att}.{p}", raw, device)
                  for p in ("q_proj", "k_proj", "v_proj", "o_proj")],
                vec(f"{att}.q_norm.weight"), vec(f"{att}.k_norm.weight"),
                vec(f"{base}.input_layernorm.weight"),
                vec(f"{base}.post_attention_layernorm.weight"), mlp))
        embed = _qweights(ts, "model.embed_tokens", raw, device)
        lm_head = None
        if not cfg.tie_word_embeddings and ts.has("lm_head.weight"):
            lm_head = _qweights(ts, "lm_head", raw, device)
        return cls(cfg, embed, layers, vec("model.norm.weight"), lm_head, dtype)

    @classmethod
    def random(cls, config: Qwen3Config, device="cuda", dtype: torch.dtype = torch.bfloat16,
               seed: int = 0, group_size: int = 64, std: float = 0.02):
        """Synthetic weights of the configured architecture, drawn directly in
        the packed int4 domain (uniform codes; per-group scales and biases of
        an N(0, std) group) - for benchmarks, where quantising billions of
        floats would only cost time."""
        gen = torch.Generator(device=device)
        gen.manual_seed(seed)
        c = config

        def qw(*shape):
            *lead, out, inn = shape
            words = torch.randint(-2**31, 2**31 - 1, (*lead, out, inn // 8), dtype=torch.int32,
                                  device=device, generator=gen)
            s = (torch.rand((*lead, out, inn // group_size), device=device, generator=gen)
                 * 0.5 + 0.75) * (std * 6.0 / 15.0)
            b = -7.5 * s
            return QuantizedWeights(s.to(dtype), b.to(dtype), group_size, 4, words)

        def ones(n):
            return torch.ones(n, dtype=dtype, device=device)

        H, D = c.hidden_size, c.head_dim
        layers = []
        for i in range(c.num_hidden_layers):
            if c.is_sparse(i):
                E, I = c.num_experts, c.moe_intermediate_size
                mlp = Moe(qw(E, H), qw(E, I, H), qw(E, I, H), qw(E, H, I),
                          num_experts_per_tok=c.num_experts_per_tok,
                          norm_topk_prob=c.norm_topk_prob)
            else:
                I = c.intermediate_size
                mlp = DenseMLP(qw(I, H), qw(I, H), qw(H, I))
            layers.append(Qwen3Layer(qw(c.num_attention_heads * D, H),
                                     qw(c.num_key_value_heads * D, H),
                                     qw(c.num_key_value_heads * D, H),
                                     qw(H, c.num_attention_heads * D),
                                     ones(D), ones(D), ones(H), ones(H), mlp))
        embed = qw(c.vocab_size, H)
        lm_head = None if c.tie_word_embeddings else qw(c.vocab_size, H)
        return cls(c, embed, layers, ones(H), lm_head, dtype)


def qwen3_30b_a3b_config(num_hidden_layers: int = 48) -> Qwen3Config:
    """Qwen3-30B-A3B's architecture (its config.json)."""
    return Qwen3Config(hidden_size=2048, num_hidden_layers=num_hidden_layers,
                       num_attention_heads=32, num_key_value_heads=4, head_dim=128,
                       vocab_size=151936, intermediate_size=6144, moe_intermediate_size=768,
                       num_experts=128, num_experts_per_tok=8, norm_topk_prob=True,
                       rms_norm_eps=1e-6, rope_theta=1000000.0, max_position_embeddings=40960,
                       tie_word_embeddings=False)

