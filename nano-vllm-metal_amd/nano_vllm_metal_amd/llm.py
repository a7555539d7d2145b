"""``LLM`` / ``SamplingParams``: batched generation over the Qwen3 model.

Mirrors the reference's high-level entry point (``llm.py:21-93``,
``sampling_params.py``) and its scheduler's loop (``engine/scheduler.py``):
requests wait in a queue; while fewer than ``max_num_seqs`` run and the page
pool has room, requests are admitted and prefilled (requests of one prompt
length together, up to ``prefill_step`` tokens per step; a longer prompt in
chunks of ``prefill_step``); then every running request decodes one
token in a single batched step; a request that reaches ``max_tokens`` (or its
end-of-sequence token) is retired and its pages freed.  Sampling follows
``layers/sampler.py``: greedy at temperature 0, else temperature with top-k
and top-p filtering.

Prompts are token-id lists, or strings when a tokenizer is given (or found in
the checkpoint directory; loaded with ``local_files_only``, no hub access).
"""

from __future__ import annotations

import time
from collections import deque
from dataclasses import dataclass, field
from typing import List, Optional, Sequence, Union

import torch

from .moe import Moe
from .qwen3 import Qwen3Model, StepInputs


@dataclass
class SamplingParams:
    """Decoding controls (``sampling_params.py``): temperature 0 is greedy."""

    max_tokens: int = 64
    temperature: float = 0.0
    top_p: float = 0.0
    top_k: Optional[int] = None
    ignore_eos: bool = False


@dataclass
class GenerationOutput:
    prompt: Union[str, List[int]]
    text: str
    token_ids: List[int] = field(default_factory=list)


@dataclass
class GenerateStats:
    prefill_tokens: int = 0
    decode_tokens: int = 0
    prefill_s: float = 0.0
    decode_s: float = 0.0
    decode_steps: int = 0


def sample(logits: torch.Tensor, sp: SamplingParams, generator=None) -> torch.Tensor:
    """Next token per row of ``logits [B, V]`` (``layers/sampler.py``)."""
    if not sp.temperature or sp.temperature <= 0:
        return torch.argmax(logits, dim=-1)
    lp = torch.log_softmax(logits.float(), dim=-1)
    if sp.top_k is not None and sp.top_k > 0:
        kth = torch.topk(lp, sp.top_k, dim=-1).values[:, -1:]
        lp = torch.where(lp < kth, torch.full_like(lp, -float("inf")), lp)
    if sp.top_p and sp.top_p > 0:
        srt, idx = torch.sort(lp, dim=-1, descending=True)
        keep = torch.cumsum(torch.exp(srt), dim=-1) < sp.top_p
        keep[:, 0] = True
        srt = torch.where(keep, srt, torch.full_like(srt, -float("inf")))
        lp = torch.full_like(lp, -float("inf")).scatter(-1, idx, srt)
    probs = torch.softmax(lp / sp.temperature, dim=-1)
    return torch.multinomial(probs, 1, generator=generator)[:, 0]


class _DecodeGraph:
    """One decode step of B requests captured in a HIP graph: static index
    buffers are refilled before each replay.  Warm-up and capture run with
    empty contexts and write only the cache's scratch page."""

    def __init__(self, model: Qwen3Model, cache, B: int, width: int):
        dev = model.device
        self.tokens = torch.zeros((B, 1), dtype=torch.long, device=dev)
        self.step = StepInputs(
            positions=torch.zeros((B,), dtype=torch.int32, device=dev),
            page_ids=torch.full((B,), cache.scratch_page, dtype=torch.int32, device=dev),
            slots=torch.zeros((B,), dtype=torch.int32, device=dev),
            block_table=torch.full((B, width), -1, dtype=torch.int32, device=dev),
            lens=torch.zeros((B,), dtype=torch.int32, device=dev), initial=False)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(2):
                model.run(self.tokens, self.step, cache)
        torch.cuda.current_stream(dev).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.logits = model.run(self.tokens, self.step, cache)

    def __call__(self, tokens: torch.Tensor, step: StepInputs) -> torch.Tensor:
        self.tokens.copy_(tokens)
        for name in ("positions", "page_ids", "slots", "block_table", "lens"):
            getattr(self.step, name).copy_(getattr(step, name))
        self.graph.replay()
        return self.logits


class _Request:
    def __init__(self, rid: int, prompt, ids: List[int], sp: SamplingParams):
        self.rid = rid
        self.prompt = prompt
        self.ids = list(ids)
        self.sp = sp
        self.out: List[int] = []
        self.done = False


class LLM:
    """``LLM(model, max_num_seqs=8, max_model_len=4096, page_size=16)``.

    ``model`` is a checkpoint directory or a ready ``Qwen3Model``."""

    def __init__(self, model: Union[str, Qwen3Model], max_num_seqs: int = 8,
                 max_model_len: int = 4096, page_size: int = 16, prefill_step: int = 2048,
                 tokenizer=None, device="cuda", dtype: torch.dtype = torch.bfloat16,
                 eos_token_id: Optional[int] = None, use_graphs: bool = True):
        if isinstance(model, Qwen3Model):
            self.model = model
        else:
            self.model = Qwen3Model.from_checkpoint(model, device=device, dtype=dtype)
            if tokenizer is None:
                tokenizer = _local_tokenizer(model)
        self.tokenizer = tokenizer
        self.max_num_seqs = max_num_seqs
        self.max_model_len = max_model_len
        self.prefill_step = prefill_step
        pages_per_seq = -(-max_model_len // page_size)
        self.pages_per_seq = pages_per_seq
        self.cache = self.model.create_kv_cache(max_num_seqs * pages_per_seq, page_size)
        # decode steps replay HIP graphs (one per batch size).  The MoE
        # workspaces are sized for the largest step first, so a captured graph
        # never refers to a buffer that a later, larger call reallocates.
        self.use_graphs = use_graphs
        self._graphs = {}
        c = self.model.config
        t_max = max(prefill_step, max_num_seqs)
        for layer in self.model.layers:
            if isinstance(layer.mlp, Moe):
                layer.mlp._workspace(t_max, c.hidden_size, c.moe_intermediate_size,
                                     c.num_experts, self.model.device)
        if eos_token_id is None and tokenizer is not None:
            eos_token_id = getattr(tokenizer, "eos_token_id", None)
        self.eos_token_id = eos_token_id
        self.stats = GenerateStats()

    def _encode(self, prompt) -> List[int]:
        if isinstance(prompt, str):
            if self.tokenizer is None:
                raise ValueError("string prompts need a tokenizer; pass token ids instead")
            return list(self.tokenizer.encode(prompt))
        return [int(t) for t in prompt]

    def _detok(self, ids: List[int]) -> str:
        return self.tokenizer.decode(ids) if self.tokenizer is not None else ""

    def _finished(self, r: _Request, tok: int) -> bool:
        if len(r.out) >= r.sp.max_tokens:
            return True
        if not r.sp.ignore_eos and self.eos_token_id is not None and tok == self.eos_token_id:
            return True
        return len(r.ids) + len(r.out) >= self.max_model_len

    def _decode_step(self, tokens: torch.Tensor, seq_ids: List[int]) -> torch.Tensor:
        """One decode step of the running requests (graph replay when enabled)."""
        m, cache = self.model, self.cache
        if not self.use_graphs:
            return m.forward(tokens, cache, seq_ids)
        step = m.prepare(cache, seq_ids, 1, width=self.pages_per_seq)
        B = len(seq_ids)
        if B not in self._graphs:
            self._graphs[B] = _DecodeGraph(m, cache, B, self.pages_per_seq)
        logits = self._graphs[B](tokens, step)
        cache.advance(seq_ids, 1)
        return logits

    def _prefill(self, batch: List[_Request]) -> List[int]:
        """Prefill requests of one prompt length together (B x L tokens, at
        most ``prefill_step``), or one long prompt in chunks; returns the first
        sampled token of each."""
        m, cache = self.model, self.cache
        for r in batch:
            cache.add(r.rid)
        L = len(batch[0].ids)
        if L <= self.prefill_step:
            toks = torch.tensor([r.ids for r in batch], dtype=torch.long, device=m.device)
            logits = m.forward(toks, cache, [r.rid for r in batch])
        else:
            (r,) = batch
            for s in range(0, L, self.prefill_step):
                chunk = torch.tensor([r.ids[s:s + self.prefill_step]], dtype=torch.long,
                                     device=m.device)
                logits = m.forward(chunk, cache, [r.rid])
        self.stats.prefill_tokens += L * len(batch)
        return [int(t) for t in sample(logits, batch[0].sp).tolist()]

    def _admit(self, waiting: deque, running: List[_Request]) -> None:
        """Admit waiting requests while a sequence slot is free, prefill them
        (equal prompt lengths batched) and move the unfinished ones to running."""
        cache = self.cache
        admitted: List[_Request] = []
        while waiting and len(running) + len(admitted) < self.max_num_seqs:
            r = waiting[0]
            need = -(-(len(r.ids) + r.sp.max_tokens) // cache.page_size)
            if need > cache.free_pages and (running or admitted):
                break
            admitted.append(waiting.popleft())
        by_len = {}
        for r in admitted:
            by_len.setdefault(len(r.ids), []).append(r)
        for L, group in by_len.items():
            per = max(1, self.prefill_step // L)
            for i in range(0, len(group), per):
                batch = group[i:i + per]
                torch.cuda.synchronize(self.model.device)
                t0 = time.perf_counter()
                toks = self._prefill(batch)
                torch.cuda.synchronize(self.model.device)
                self.stats.prefill_s += time.perf_counter() - t0
                for r, tok in zip(batch, toks):
                    r.out.append(tok)
                    if self._finished(r, tok):
                        r.done = True
                        cache.free(r.rid)
                    else:
                        running.append(r)

    def generate(self, prompts: Union[str, Sequence], sampling_params: Optional[SamplingParams] = None
                 ) -> List[GenerationOutput]:
        if isinstance(prompts, (str,)) or (len(prompts) and isinstance(prompts[0], int)):
            prompts = [prompts]
        sp = sampling_params or SamplingParams()
        reqs = [_Request(i, p, self._encode(p), sp) for i, p in enumerate(prompts)]
        for r in reqs:
            if not r.ids:
                raise ValueError("empty prompt")
            if len(r.ids) >= self.max_model_len:
                raise ValueError(f"prompt of {len(r.ids)} tokens exceeds max_model_len")
        waiting = deque(reqs)
        running: List[_Request] = []
        m, cache = self.model, self.cache
        while waiting or running:
            self._admit(waiting, running)
            if not running:
                continue
            torch.cuda.synchronize(m.device)
            t0 = time.perf_counter()
            last = torch.tensor([[r.out[-1]] for r in running], dtype=torch.long, device=m.device)
            logits = self._decode_step(last, [r.rid for r in running])
            nxt = sample(logits, sp).tolist()
            self.stats.decode_s += time.perf_counter() - t0
            self.stats.decode_steps += 1
            self.stats.decode_tokens += len(running)
            still = []
            for r, tok in zip(running, nxt):
                r.out.append(int(tok))
                if self._finished(r, int(tok)):
                    r.done = True
                    cache.free(r.rid)
                else:
                    still.append(r)
            running = still
        return [GenerationOutput(r.prompt, self._detok(r.out), r.out) for r in reqs]


def _local_tokenizer(path):
    try:
        from transformers import AutoTokenizer

        return AutoTokenizer.from_pretrained(str(path), local_files_only=True)
    except Exception:  # no tokenizer files in the checkpoint: token-id prompts only
        return None
