"""The full 48-layer Qwen3-30B-A3B-shaped model at the end-to-end benchmark's
own size: 32 concurrent requests of 1024 random tokens, 256 greedy tokens
each, through LLM.generate with the paged KV cache (random int4 weights).

The reference checks continuous batching against full forwards
(tests/test_batching.py:256-318 of the reference).  There is no float32
reference forward at this size here (it would take hours on the CPU), so the
run is checked through properties that a wrong batch composition, a wrong
page or a corrupted step would break:

* every request produces its 256 tokens and every KV page is free afterwards;
* requests re-run alone (one sequence, other decode launch shapes and other
  attention split counts) reproduce the batch's greedy tokens; where the two
  runs part, the batch's token is within 4 bf16 ulps of the maximum of the
  lone sequence's logits at that position (recomputed by one forward over
  prompt and tokens), i.e. a near-tie that summation order can flip - the
  same bar as the 2-layer 30B-dimension test against the float32 reference;
* those logits are finite.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _row_ulp(v: torch.Tensor) -> float:
    top = float(v.float().abs().max().clamp_min(2.0 ** -100))
    return 2.0 ** (np.floor(np.log2(top)) - 7)


def test_generate_48_layers_32_requests_of_1024_tokens():
    from nano_vllm_metal_amd import LLM, Qwen3Model, SamplingParams, qwen3_30b_a3b_config

    n_seqs, L, gen = 32, 1024, 256
    cfg = qwen3_30b_a3b_config(48)
    m = Qwen3Model.random(cfg, device=DEV, seed=7)
    rng = np.random.default_rng(3)
    prompts = [rng.integers(0, cfg.vocab_size, L).tolist() for _ in range(n_seqs)]
    sp = SamplingParams(max_tokens=gen, ignore_eos=True)
    llm = LLM(m, max_num_seqs=n_seqs, max_model_len=L + gen + 16, page_size=16,
              prefill_step=8 * L)
    outs = llm.generate(prompts, sp)
    torch.cuda.synchronize()
    print(f"config 5: {n_seqs} x {L} prompts, {gen} tokens each generated", flush=True)
    assert [len(o.token_ids) for o in outs] == [gen] * n_seqs
    assert llm.cache.free_pages == llm.cache.num_pages
    del llm

    solo = LLM(m, max_num_seqs=1, max_model_len=L + gen + 16, page_size=16, prefill_step=8 * L)
    for i in (0, 13, 31):
        batch = outs[i].token_ids
        alone = solo.generate([prompts[i]], sp)[0].token_ids
        assert solo.cache.free_pages == solo.cache.num_pages
        d = next((j for j in range(gen) if batch[j] != alone[j]), gen)
        # the lone sequence's logits at the first position the runs differ
        # (or at the last one), recomputed in one forward
        j = min(d, gen - 1)
        cache = m.create_kv_cache(-(-(L + gen) // 16), page_size=16)
        cache.add(0)
        toks = torch.tensor([prompts[i] + alone[:j]], device=DEV)
        logits = m.forward(toks, cache, [0])[0].float()
        torch.cuda.synchronize()
        assert bool(torch.isfinite(logits).all()), f"request {i}: non-finite logits"
        ulp = _row_ulp(logits)
        gap_alone = float(logits.max() - logits[alone[j]]) / ulp
        gap_batch = float(logits.max() - logits[batch[j]]) / ulp
        print(f"request {i}: alone == batch for the first {d} of {gen} tokens; at token {j} "
              f"the lone run's token is {gap_alone:.2f} ulps and the batch's {gap_batch:.2f} "
              f"ulps below the maximum logit", flush=True)
        assert gap_alone <= 4.0
        if d < gen:
            assert gap_batch <= 4.0, f"request {i}: batch token {batch[j]} is not a near-tie"
        del cache
